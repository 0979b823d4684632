"""Qwen2 decoder forward on the MI355X: HIP kernels for every token-wise op and for attention.

Interface follows nanoserve/model.py (ModelConfig :26-56, LayerWeights :67-114, SeqInput :117-129,
DecodeMeta :132-137, Qwen2Model :154-367) so the engine, scheduler, KV manager and graph runners call it
the same way. The math of one layer on N flattened tokens (nanoserve/model.py:223-260, fused path):

    h      = rms_norm(x, ln1)
    q,k,v  = rope_qkv(h @ [Wq;Wk;Wv]^T + [bq;bk;bv], cos, sin) + K/V stored at slots
    o      = paged attention over each row's pages                       (kernels/paged_attention.py)
    h, x   = rms_norm(o @ Wo^T, ln2, residual=x)
    x      = x + silu_mul(h @ [Wg;Wu]^T) @ Wd^T

For decode-sized bf16 batches (M <= 64) each projection is one skinny HIP GEMM with the neighbouring op in
its epilogue (kernels/linear.py): QKV + bias + RoPE + KV write; O + residual + RMSNorm statistics;
gate/up + SiLU*mul with ln2 applied on load; down + residual + statistics for the NEXT RMSNorm (the next
layer's ln1, or the final norm after the last layer), applied on load by its consumer -- so a decode layer
is 4 GEMM launches and 1 attention launch. Larger bf16 batches (prefill chunks, mixed steps, verify
batches) use the tiled MFMA GEMM (SiLU*mul fused into gate/up) or, up to 192 rows, the token-blocked
skinny kernels, plus the standalone HIP RMSNorm and RoPE kernels; every one rounds where PyTorch's unfused
ops round. fp32 (the correctness configuration) runs its projections through torch's F.linear.

Attention reads K/V in place from the pages rope_qkv has just written. One-token decode rows (DecodeMeta)
go through the paged decode kernel; the tokens of prefill / chunked-prefill sequences go through the paged
chunked-prefill kernel (bf16), where token j of a sequence with ctx_len cached tokens sees keys
0 .. ctx_len + j: exactly the causal offset mask of nanoserve/model.py:292-309. In fp32 (the correctness
configuration) those tokens run as decode rows with context ctx_len + j + 1, the same mask.

Only the HIP path exists here: a CPU tensor, the contiguous cache or a missing kernel library raise. The
unfused PyTorch restatement (the CPU oracle used by the tests) lives outside this package.
"""
from __future__ import annotations

import copy
import json
from dataclasses import dataclass
from pathlib import Path

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class ModelConfig:
    vocab_size: int
    hidden_size: int
    n_layers: int
    n_heads: int            # query heads
    n_kv_heads: int         # key/value heads (GQA)
    head_dim: int
    intermediate_size: int  # MLP width
    rope_theta: float
    rms_norm_eps: float
    tie_word_embeddings: bool

    @classmethod
    def from_hf_config(cls, d: dict) -> "ModelConfig":
        rope_theta = d.get("rope_theta") or (d.get("rope_parameters") or {}).get("rope_theta")
        return cls(vocab_size=d["vocab_size"], hidden_size=d["hidden_size"], n_layers=d["num_hidden_layers"],
                   n_heads=d["num_attention_heads"], n_kv_heads=d["num_key_value_heads"],
                   head_dim=d.get("head_dim") or d["hidden_size"] // d["num_attention_heads"],
                   intermediate_size=d["intermediate_size"], rope_theta=float(rope_theta),
                   rms_norm_eps=d["rms_norm_eps"], tie_word_embeddings=d.get("tie_word_embeddings", False))

    @classmethod
    def from_pretrained(cls, folder: str) -> "ModelConfig":
        return cls.from_hf_config(json.loads((_local_folder(folder) / "config.json").read_text()))

    def kv_bytes_per_token(self, dtype: torch.dtype) -> int:
        """KV memory of one token: every layer stores one K and one V vector per KV head."""
        return self.n_layers * 2 * self.n_kv_heads * self.head_dim * torch.finfo(dtype).bits // 8


# Architectures of the benchmark configurations (Qwen2.5 shapes; weights are random-init).
QWEN25_0_5B = ModelConfig(vocab_size=151936, hidden_size=896, n_layers=24, n_heads=14, n_kv_heads=2, head_dim=64,
                          intermediate_size=4864, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
QWEN25_1_5B = ModelConfig(vocab_size=151936, hidden_size=1536, n_layers=28, n_heads=12, n_kv_heads=2, head_dim=128,
                          intermediate_size=8960, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
QWEN25_3B = ModelConfig(vocab_size=151936, hidden_size=2048, n_layers=36, n_heads=16, n_kv_heads=2, head_dim=128,
                        intermediate_size=11008, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)


def _local_folder(name: str) -> Path:
    p = Path(name)
    if not p.is_dir():
        raise FileNotFoundError(f"{name}: a local model folder (config.json + *.safetensors) is required; "
                                "this build never downloads")
    return p


@dataclass
class LayerWeights:
    ln1: torch.Tensor
    q_w: torch.Tensor
    q_b: torch.Tensor
    k_w: torch.Tensor
    k_b: torch.Tensor
    v_w: torch.Tensor
    v_b: torch.Tensor
    o_w: torch.Tensor
    ln2: torch.Tensor
    gate_w: torch.Tensor
    up_w: torch.Tensor
    down_w: torch.Tensor
    qkv_w: torch.Tensor | None = None     # merged [q; k; v] rows (per-matrix fields become views)
    qkv_b: torch.Tensor | None = None
    gate_up_w: torch.Tensor | None = None  # merged [gate; up] rows
    # fragment-packed copies for decode-sized products (kernels/linear.py PackedWeight), bf16 on the GPU
    qkv_p: object | None = None
    o_p: object | None = None
    gate_up_p: object | None = None
    down_p: object | None = None

    HF_NAMES = {
        "ln1": "input_layernorm.weight",
        "q_w": "self_attn.q_proj.weight", "q_b": "self_attn.q_proj.bias",
        "k_w": "self_attn.k_proj.weight", "k_b": "self_attn.k_proj.bias",
        "v_w": "self_attn.v_proj.weight", "v_b": "self_attn.v_proj.bias",
        "o_w": "self_attn.o_proj.weight",
        "ln2": "post_attention_layernorm.weight",
        "gate_w": "mlp.gate_proj.weight", "up_w": "mlp.up_proj.weight", "down_w": "mlp.down_proj.weight",
    }

    @classmethod
    def from_state_dict(cls, sd: dict, i: int) -> "LayerWeights":
        return cls(**{f: sd[f"model.layers.{i}.{hf}"] for f, hf in cls.HF_NAMES.items()})

    def merge(self) -> None:
        """Merged QKV and gate/up matrices (one GEMM each); the per-matrix fields become row views of them,
        so nothing is stored twice (nanoserve/model.py:101-114)."""
        if self.qkv_w is not None:
            return
        nq, nk, ng = self.q_w.shape[0], self.k_w.shape[0], self.gate_w.shape[0]
        self.qkv_w = torch.cat([self.q_w, self.k_w, self.v_w])
        self.q_w, self.k_w, self.v_w = self.qkv_w[:nq], self.qkv_w[nq:nq + nk], self.qkv_w[nq + nk:]
        self.qkv_b = torch.cat([self.q_b, self.k_b, self.v_b])
        self.q_b, self.k_b, self.v_b = self.qkv_b[:nq], self.qkv_b[nq:nq + nk], self.qkv_b[nq + nk:]
        self.gate_up_w = torch.cat([self.gate_w, self.up_w])
        self.gate_w, self.up_w = self.gate_up_w[:ng], self.gate_up_w[ng:]


@dataclass
class SeqInput:
    """One sequence's slice of a batched step (nanoserve/model.py:117-129). Paged only: `block_table` =
    this request's block ids (a list, or an int tensor on the device; may be None for a fresh prefill, whose
    pages are then read off the slot mapping), `ctx_len` = tokens already stored before this step."""
    n_tokens: int
    cache: object | None = None
    block_table: torch.Tensor | None = None
    ctx_len: int = 0
    use_kernel: bool = False      # a one-token decode handled through DecodeMeta


@dataclass
class DecodeMeta:
    """Built once per step for all one-token decode rows (nanoserve/model.py:132-137)."""
    token_idx: torch.Tensor       # [Bd] positions of their tokens in the flattened batch
    block_tables: torch.Tensor    # [Bd, max_blocks] int32
    context_lens: torch.Tensor    # [Bd] int32, including this step's token
    all_rows: bool = False        # token_idx is arange(N): rows map 1:1 to the step's tokens (no gather)
    pairs: torch.Tensor | None = None   # [Bd] int32: rows sharing a block table, run together (pair_rows)


def random_state_dict(cfg: ModelConfig, seed: int = 0, dtype: torch.dtype = torch.bfloat16,
                      device: str | torch.device = "cpu") -> dict[str, torch.Tensor]:
    """Random-init Qwen2 weights under HF names, drawn on the CPU in fp32 with one seeded generator in HF
    order (embed_tokens first, then each layer's tensors in LayerWeights.HF_NAMES order, then the final
    norm): matrices and biases ~ N(0, 0.02), norm weights = 1, LM head tied to the embedding. Identical
    values for the CPU oracle and the GPU, whatever the dtype."""
    g = torch.Generator(device="cpu").manual_seed(seed)

    def normal(*shape):
        t = torch.empty(*shape, dtype=torch.float32)
        t.normal_(0.0, 0.02, generator=g)
        return t.to(dtype).to(device)

    H, I, hd = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    sd = {"model.embed_tokens.weight": normal(cfg.vocab_size, H)}
    shapes = {"q_w": (cfg.n_heads * hd, H), "q_b": (cfg.n_heads * hd,), "k_w": (cfg.n_kv_heads * hd, H),
              "k_b": (cfg.n_kv_heads * hd,), "v_w": (cfg.n_kv_heads * hd, H), "v_b": (cfg.n_kv_heads * hd,),
              "o_w": (H, cfg.n_heads * hd), "gate_w": (I, H), "up_w": (I, H), "down_w": (H, I)}
    for i in range(cfg.n_layers):
        for field, hf in LayerWeights.HF_NAMES.items():
            name = f"model.layers.{i}.{hf}"
            if field in ("ln1", "ln2"):
                sd[name] = torch.ones(H, dtype=dtype, device=device)
            else:
                sd[name] = normal(*shapes[field])
    sd["model.norm.weight"] = torch.ones(H, dtype=dtype, device=device)
    if not cfg.tie_word_embeddings:
        sd["lm_head.weight"] = normal(cfg.vocab_size, H)
    return sd


class Qwen2Model:
    """Weights + forward; no nn.Module (nothing is trained)."""

    fused = True

    def __init__(self, cfg: ModelConfig, state_dict: dict[str, torch.Tensor], pack: bool | None = None):
        """pack: also store the projection weights fragment-packed for decode-sized steps (default: bf16 on the
        GPU; the packed copies add the size of the layer and LM-head weights once more)."""
        self.cfg = cfg
        self.embed = state_dict["model.embed_tokens.weight"]
        self.norm = state_dict["model.norm.weight"]
        self.lm_head = self.embed if cfg.tie_word_embeddings else state_dict["lm_head.weight"]
        self.layers = [LayerWeights.from_state_dict(state_dict, i) for i in range(cfg.n_layers)]
        for layer in self.layers:
            layer.merge()
        self.device = self.embed.device
        self.dtype = self.embed.dtype
        # RoPE inverse frequencies, fp32, computed on the CPU like HF, then moved
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, dtype=torch.float) / cfg.head_dim))
        self.inv_freq = inv.to(self.device)
        self.lm_head_p = None
        if pack is None:
            pack = self.dtype == torch.bfloat16 and self.device.type == "cuda"
        if pack:
            self._pack()

    def _pack(self) -> None:
        """Fragment-packed copies of every projection weight (kernels/linear.py PackedWeight)."""
        from nanoserve_amd.kernels.linear import PACK_GATE_UP, PACK_ROPE, PackedWeight
        cfg = self.cfg
        if cfg.hidden_size % 32 or cfg.intermediate_size % 32 or (cfg.n_heads * cfg.head_dim) % 32:
            return
        for layer in self.layers:
            layer.qkv_p = PackedWeight(layer.qkv_w, PACK_ROPE, cfg.head_dim) if cfg.head_dim in (64, 128) else None
            layer.o_p = PackedWeight(layer.o_w)
            layer.gate_up_p = PackedWeight(layer.gate_up_w, PACK_GATE_UP)
            # down (K = intermediate > 2048): its packed plan would slice K, and the slice merge costs more
            # than the row-major kernel's streaming, so it stays row-major only
            if cfg.intermediate_size <= 2048:
                layer.down_p = PackedWeight(layer.down_w)
        self.lm_head_p = PackedWeight(self.lm_head.contiguous())

    @classmethod
    def from_pretrained(cls, folder: str, device: str | torch.device = "cuda",
                        dtype: torch.dtype = torch.bfloat16) -> "Qwen2Model":
        """Load a local HF folder (config.json + *.safetensors); converts one tensor at a time."""
        from safetensors.torch import load_file
        path = _local_folder(folder)
        cfg = ModelConfig.from_pretrained(str(path))
        raw: dict[str, torch.Tensor] = {}
        for f in sorted(path.glob("*.safetensors")):
            raw.update(load_file(str(f), device="cpu"))
        sd = {k: raw.pop(k).to(dtype).to(device) for k in list(raw)}
        return cls(cfg, sd)

    def with_fused_ops(self) -> "Qwen2Model":
        """The HIP path is always fused; returns a shallow copy sharing the weights (reference API)."""
        m = copy.copy(self)
        m.fused = True
        return m

    def named_weights(self) -> dict[str, torch.Tensor]:
        out = {"model.embed_tokens.weight": self.embed, "model.norm.weight": self.norm}
        if not self.cfg.tie_word_embeddings:
            out["lm_head.weight"] = self.lm_head
        for i, layer in enumerate(self.layers):
            for field, hf in LayerWeights.HF_NAMES.items():
                out[f"model.layers.{i}.{hf}"] = getattr(layer, field)
        return out

    # ---------------------------------------------------------------------------------------- pieces
    def _require_gpu(self) -> None:
        if self.device.type != "cuda":
            raise ValueError("Qwen2Model runs the HIP kernels: put the weights on the GPU")

    def final_norm(self, x: torch.Tensor) -> torch.Tensor:
        from nanoserve_amd.kernels.fused import rms_norm
        return rms_norm(x, self.norm, self.cfg.rms_norm_eps)

    def rope(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """cos/sin [1, T, head_dim] in the model dtype (nanoserve/model.py:212-217)."""
        freqs = positions[None, :, None].float() * self.inv_freq.to(device=positions.device, dtype=torch.float)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(self.dtype), emb.sin().to(self.dtype)

    def _pre(self, i: int, x: torch.Tensor, cos, sin, paged=None, slot_mapping=None):
        """RMSNorm, merged QKV GEMM, RoPE + paged K/V write. x [1, N, H] -> q [1,N,nh,hd], k/v [1,N,nkv,hd]."""
        from nanoserve_amd.kernels.fused import rms_norm
        h = rms_norm(x, self.layers[i].ln1, self.cfg.rms_norm_eps)[0]
        return self._qkv(i, h, cos, sin, paged, slot_mapping)

    def _qkv(self, i: int, h: torch.Tensor, cos, sin, paged=None, slot_mapping=None):
        """QKV projection (+ bias) of the normed activations h [N, H], RoPE, K/V stored at the slots."""
        from nanoserve_amd.kernels.linear import linear_rope_qkv
        layer, cfg = self.layers[i], self.cfg
        q, k, v = linear_rope_qkv(h, layer.qkv_p or layer.qkv_w, layer.qkv_b, cos[0], sin[0], cfg.n_heads, cfg.n_kv_heads,
                                  cfg.head_dim, paged.k[i] if paged is not None else None,
                                  paged.v[i] if paged is not None else None, slot_mapping)
        return q[None], k[None], v[None]

    def _mlp(self, i: int, x: torch.Tensor, o: torch.Tensor, next_norm: torch.Tensor | None):
        """o_proj + residual + RMSNorm, SwiGLU MLP + residual; with next_norm, the following RMSNorm (the
        next layer's ln1 or the final norm) is applied in the same epilogue. x, o 2-D -> (h_next, x)."""
        from nanoserve_amd.kernels.linear import linear_residual_rms_norm, linear_silu_mul
        layer, eps = self.layers[i], self.cfg.rms_norm_eps
        h, x = linear_residual_rms_norm(o, layer.o_p or layer.o_w, x, layer.ln2, eps)
        a = linear_silu_mul(h, layer.gate_up_p or layer.gate_up_w)
        return linear_residual_rms_norm(a, layer.down_p or layer.down_w, x, next_norm, eps)

    def _post(self, i: int, x: torch.Tensor, o: torch.Tensor) -> torch.Tensor:
        """o_proj + residual (fused into the norm), RMSNorm, SwiGLU MLP + residual. x [1,N,H], o [1,N,nh*hd]."""
        return self._mlp(i, x[0], o[0], None)[1][None]

    def _attend(self, i: int, q, k, v, seqs: list[SeqInput], paged=None, decode_meta=None,
                out: torch.Tensor | None = None, slot_mapping: torch.Tensor | None = None) -> torch.Tensor:
        """Attention of layer i for the step's flattened tokens; q [1, N, nh, hd]. Returns [1, N, nh*hd]
        (written into `out` if given). Decode rows come from decode_meta; every other sequence's tokens are
        rows with causal-offset contexts (see the module docstring)."""
        from nanoserve_amd.kernels.paged_attention import paged_attention_decode, paged_attention_decode_rows
        if paged is None:
            raise ValueError("the HIP attention path reads the paged KV cache: pass `paged`")
        N, nh, hd = q.shape[1], q.shape[2], q.shape[3]
        scale = hd ** -0.5
        if decode_meta is not None and decode_meta.all_rows:
            o = paged_attention_decode(q[0], paged.k[i], paged.v[i], decode_meta.block_tables,
                                       decode_meta.context_lens, scale, pairs=decode_meta.pairs)
            if out is None:
                return o.view(1, N, nh * hd)
            out[0].copy_(o.view(N, nh * hd))
            return out
        o_all = out if out is not None else torch.empty(1, N, nh * hd, device=q.device, dtype=q.dtype)
        pre = self._prefill_meta(seqs, paged, slot_mapping, q.dtype)
        if decode_meta is not None and pre is not None and pre[0] == "chunks":
            # decode rows and chunks in one launch (their workgroups share the grid)
            from nanoserve_amd.kernels.paged_attention import paged_attention_mixed
            _, tables, info, max_new, max_kv = pre
            paged_attention_mixed(q[0], paged.k[i], paged.v[i], tables, info, max_new, max_kv,
                                  decode_meta.block_tables, decode_meta.context_lens, decode_meta.token_idx, scale,
                                  out=o_all[0].view(N, nh, hd))
            return o_all
        if decode_meta is not None:   # the decode rows' queries and outputs addressed in place
            paged_attention_decode_rows(q[0], paged.k[i], paged.v[i], decode_meta.block_tables,
                                        decode_meta.context_lens, decode_meta.token_idx, scale,
                                        out=o_all[0].view(N, nh, hd))
        if pre is not None and pre[0] == "chunks":
            from nanoserve_amd.kernels.paged_attention import paged_attention_prefill
            _, tables, info, max_new, max_kv = pre
            paged_attention_prefill(q[0], paged.k[i], paged.v[i], tables, info, max_new, max_kv, scale,
                                    out=o_all[0].view(N, nh, hd))
        elif pre is not None:
            _, idx, tables, lens = pre
            o_pf = paged_attention_decode(q[0][idx], paged.k[i], paged.v[i], tables, lens, scale)
            o_all[0].index_copy_(0, idx, o_pf.reshape(o_pf.shape[0], -1))
        return o_all

    def _prefill_meta(self, seqs: list[SeqInput], paged, slot_mapping, dtype: torch.dtype):
        """Attention inputs of the step's non-decode tokens (prefills and chunk continuations), cached per
        step (all layers share them):
          bf16: ("chunks", tables int32 [S, W], seq_info int32 [S, 4], max_new, max_kv) for the chunked-prefill
                kernel;
          fp32: ("rows", token index, tables [n, W], context lengths [n]) -- one decode row per token, token j
                of a sequence with ctx_len cached tokens seeing ctx_len + j + 1 tokens."""
        cache = getattr(self, "_rows_cache", None)
        if cache is not None and cache[0] is seqs and cache[1] is slot_mapping:
            return cache[2]
        from nanoserve_amd.kernels.paged_attention import prefill_seq_info
        dev, bs = self.device, paged.block_size
        tabs, starts, news, ctxs = [], [], [], []
        start = 0
        for s in seqs:
            T = s.n_tokens
            if not s.use_kernel and T > 0:
                n_pages = -(-(s.ctx_len + T) // bs)
                if isinstance(s.block_table, list):
                    bt = torch.tensor(s.block_table[:n_pages], dtype=torch.int32, device=dev)
                elif s.block_table is not None:
                    bt = s.block_table.to(device=dev, dtype=torch.int32)[:n_pages]
                    if bt.shape[0] < n_pages:
                        raise ValueError(f"block_table holds {bt.shape[0]} blocks, {n_pages} needed")
                elif s.ctx_len == 0:
                    if slot_mapping is None:
                        raise ValueError("a fresh prefill without block_table needs slot_mapping")
                    bt = (slot_mapping[start:start + T:bs] // bs).to(torch.int32)
                else:
                    raise ValueError("a continuation chunk (ctx_len > 0) needs its block_table")
                tabs.append(bt)
                starts.append(start)
                news.append(T)
                ctxs.append(s.ctx_len)
            start += T
        if not tabs:
            meta = None
        else:
            width = max(bt.shape[0] for bt in tabs)
            padded = [F.pad(bt, (0, width - bt.shape[0])) for bt in tabs]
            if dtype == torch.bfloat16:
                meta = ("chunks", torch.stack(padded).contiguous(), prefill_seq_info(starts, news, ctxs, dev), max(news),
                        max(c + t for c, t in zip(ctxs, news)))
            else:
                idx = torch.cat([torch.arange(a, a + t, device=dev) for a, t in zip(starts, news)])
                lens = torch.cat([torch.arange(c + 1, c + t + 1, device=dev, dtype=torch.int32)
                                  for c, t in zip(ctxs, news)])
                tables = torch.cat([bt[None].expand(t, width) for bt, t in zip(padded, news)]).contiguous()
                meta = ("rows", idx, tables, lens)
        self._rows_cache = (seqs, slot_mapping, meta)
        return meta

    @torch.inference_mode()
    def forward_batch(self, token_ids: torch.Tensor, positions: torch.Tensor, seqs: list[SeqInput],
                      logits="last", paged=None, slot_mapping: torch.Tensor | None = None,
                      decode_meta: DecodeMeta | None = None, prefill_meta: tuple | None = None,
                      greedy_out: torch.Tensor | None = None) -> torch.Tensor:
        """One forward pass over several sequences (prefilling, continuing a chunked prefill on a cached
        context, or decoding one token). token_ids/positions: [N] in `seqs` order. Returns logits
        [len(seqs), vocab] for each sequence's last token ("last"), [N, vocab] ("all"), or the rows of an
        index tensor. prefill_meta: the chunked-prefill kernel's inputs already on the device, ("chunks",
        tables int32 [S, W], seq_info int32 [S, 4], max_new, max_kv) -- the non-decode rows are then described
        by them alone (a captured mixed step), and `seqs` only has to cover the rows. greedy_out (int64, one
        entry per returned row; device or pinned host memory) receives the rows' argmax."""
        self._require_gpu()
        if paged is None:
            raise ValueError("the HIP path needs the paged KV cache (`paged` + `slot_mapping`)")
        assert sum(s.n_tokens for s in seqs) == token_ids.shape[0], "seqs must cover token_ids exactly"
        self._rows_cache = None if prefill_meta is None else (seqs, slot_mapping, prefill_meta)
        from nanoserve_amd.kernels.fused import embed_rope, rms_norm
        from nanoserve_amd.kernels.linear import SKINNY_MAX_M, NormedRows
        L, eps = self.cfg.n_layers, self.cfg.rms_norm_eps
        # embedding rows and RoPE tables in one launch; a decode-sized bf16 batch also gets the first
        # RMSNorm's row statistics, so layer 0's QKV projection normalises on load like every later layer
        stats = self.dtype == torch.bfloat16 and token_ids.shape[0] <= SKINNY_MAX_M
        x, cos, sin, sumsq = embed_rope(token_ids.contiguous(), positions.contiguous(), self.embed, self.inv_freq,
                                        self.cfg.head_dim, row_stats=stats)
        cos, sin = cos[None], sin[None]
        h = NormedRows(x, sumsq, self.layers[0].ln1, eps) if stats else rms_norm(x, self.layers[0].ln1, eps)
        for i in range(L):
            q, k, v = self._qkv(i, h, cos, sin, paged, slot_mapping)
            o = self._attend(i, q, k, v, seqs, paged, decode_meta, slot_mapping=slot_mapping)[0]
            next_norm = self.layers[i + 1].ln1 if i + 1 < L else self.norm
            h, x = self._mlp(i, x, o, next_norm)       # h: the next layer's normed input / the final norm
        self._rows_cache = None
        return self.lm_head_rows(h, seqs, logits, greedy_out)

    def lm_head_rows(self, x, seqs: list[SeqInput], logits="last", greedy_out: torch.Tensor | None = None) -> torch.Tensor:
        """Final-normed hidden states ([1, N, H] / [N, H] tensor, or a NormedRows) -> logits of the requested
        rows; with `greedy_out` (int64 [rows]) their argmax is written there too (fused into the LM head's
        launch where the kernel takes the shape)."""
        from nanoserve_amd.kernels.fused import gather_rows
        from nanoserve_amd.kernels.linear import NormedRows, linear, linear_argmax
        if isinstance(x, torch.Tensor) and x.dim() == 3:
            x = x[0]
        idx = None
        if isinstance(logits, torch.Tensor):
            idx = logits
        elif logits == "last":
            ends, acc = [], -1
            for s in seqs:
                acc += s.n_tokens
                ends.append(acc)
            idx = torch.tensor(ends, dtype=torch.int64, device=x.device)   # each sequence's last row
        if idx is not None:
            x = x.rows(idx) if isinstance(x, NormedRows) else gather_rows(x, idx)
        # The packed LM head (up to 64 rows) and the row-major persistent one (up to 32 rows, K <= 2048) run on
        # persistent workgroups that normalise their activation fragments once, so they take the NormedRows
        # itself; beyond that every 64-row tile would repeat the row-statistics prologue, so the final norm is
        # materialised once instead.
        if isinstance(x, NormedRows):
            packed = self.lm_head_p is not None and x.r.shape[0] <= 64
            if not packed and (x.r.shape[0] > 32 or x.r.shape[1] > 2048):
                x = x.tensor()
        else:
            x = x.contiguous()
        head = self.lm_head_p or self.lm_head
        if greedy_out is not None:
            return linear_argmax(x, head, greedy_out)
        return linear(x, head)

    def forward(self, token_ids: torch.Tensor, positions: torch.Tensor, cache=None, logits: str = "last"):
        """ONE sequence, the single-request API (nanoserve/model.py:364-367), on the paged path. `cache` is a
        kv_cache.SequenceKVCache whose `length` stored tokens precede token_ids (it advances by T), or None
        for a fresh sequence, run in a temporary pool of its own. Returns what forward_batch returns for one
        sequence: [1, vocab] ("last") or [T, vocab] ("all")."""
        from nanoserve_amd.kv_cache import SequenceKVCache
        T = int(token_ids.shape[0])
        if cache is None:
            cache = SequenceKVCache(self.cfg, T, self.device, self.dtype)
        table = cache.table
        if table.num_tokens + T > cache.max_seq_len:
            raise ValueError(f"{table.num_tokens} cached + {T} new tokens exceed the cache's {cache.max_seq_len}")
        slots = torch.tensor(table.slots(T), device=self.device)
        seq = SeqInput(T, ctx_len=table.num_tokens, block_table=table.blocks)
        out = self.forward_batch(token_ids.to(self.device), positions.to(self.device), [seq], logits=logits,
                                 paged=cache.pool, slot_mapping=slots)
        table.commit(T)
        return out

"""CPU restatement of nanoserve's Qwen2 forward on its unfused PyTorch path.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Follows nanoserve/model.py: rms_norm :140-146,
rotate_half :149-151, inv_freq :168, rope tables :212-217, unfused _pre :236-248 (separate q/k/v
projections with biases, q*cos + rotate_half(q)*sin), _post :258-260 (x + o_proj, RMSNorm, SwiGLU MLP,
residual), attention per sequence :283-318 (SDPA; is_causal for a fresh multi-token prefill, explicit
causal-offset mask + repeat_interleave for several new tokens on a cached context, no mask for one decode
token), final norm + LM head on the last row of each sequence :351-362 — selective batching: projections
run once over all of the step's tokens, attention once per sequence.

Caches here are per sequence and contiguous ([L, n_kv, S, hd]); the paged layout is an addressing
choice the tests check separately (paged == contiguous is one of the reference's own gates,
tests/test_paged_engine.py:66-77).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from oracle import ops


@dataclass
class SeqCache:
    k: torch.Tensor        # [L, n_kv, S, hd]
    v: torch.Tensor
    length: int = 0
    tokens: list[int] = field(default_factory=list)


class OracleModel:
    def __init__(self, cfg, state_dict: dict[str, torch.Tensor], dtype: torch.dtype = torch.float32):
        self.cfg = cfg
        self.dtype = dtype
        sd = {k: v.detach().to("cpu", dtype) for k, v in state_dict.items()}
        self.embed = sd["model.embed_tokens.weight"]
        self.norm = sd["model.norm.weight"]
        self.lm_head = self.embed if cfg.tie_word_embeddings else sd["lm_head.weight"]
        names = ["input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.q_proj.bias",
                 "self_attn.k_proj.weight", "self_attn.k_proj.bias", "self_attn.v_proj.weight",
                 "self_attn.v_proj.bias", "self_attn.o_proj.weight", "post_attention_layernorm.weight",
                 "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"]
        self.layers = [[sd[f"model.layers.{i}.{n}"] for n in names] for i in range(cfg.n_layers)]

    def new_cache(self, max_len: int) -> SeqCache:
        c = self.cfg
        shape = (c.n_layers, c.n_kv_heads, max_len, c.head_dim)
        return SeqCache(torch.zeros(shape, dtype=self.dtype), torch.zeros(shape, dtype=self.dtype))

    @torch.inference_mode()
    def step(self, batch: list[tuple[SeqCache, list[int]]], all_logits: bool = False) -> torch.Tensor:
        """One step over several sequences; each feeds `tokens` at positions cache.length ... Returns the
        logits of each sequence's last token [B, V] (or of every token if all_logits)."""
        cfg = self.cfg
        hd, nh, nkv = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
        toks, pos, spans = [], [], []
        for cache, t in batch:
            spans.append((len(toks), len(t)))
            toks += t
            pos += list(range(cache.length, cache.length + len(t)))
        x = F.embedding(torch.tensor(toks), self.embed)
        cos, sin = ops.rope_tables(torch.tensor(pos), hd, cfg.rope_theta, self.dtype)
        eps = cfg.rms_norm_eps
        for li, (ln1, qw, qb, kw, kb, vw, vb, ow, ln2, gw, uw, dw) in enumerate(self.layers):
            h = ops.rms_norm(x, ln1, eps)
            N = h.shape[0]
            q = self.rope(li, F.linear(h, qw, qb).view(N, nh, hd), cos, sin)
            k = self.rope(li, F.linear(h, kw, kb).view(N, nkv, hd), cos, sin)
            v = F.linear(h, vw, vb).view(N, nkv, hd)
            o = torch.empty(N, nh * hd, dtype=self.dtype)
            for (cache, _), (s0, T) in zip(batch, spans):
                L0 = cache.length
                cache.k[li, :, L0:L0 + T] = k[s0:s0 + T].transpose(0, 1)
                cache.v[li, :, L0:L0 + T] = v[s0:s0 + T].transpose(0, 1)
                ks = cache.k[li, :, :L0 + T].transpose(0, 1)
                vs = cache.v[li, :, :L0 + T].transpose(0, 1)
                o[s0:s0 + T] = self.attend(li, q[s0:s0 + T], ks, vs, L0).reshape(T, nh * hd)
            x = x + F.linear(o, ow)
            h = ops.rms_norm(x, ln2, eps)
            x = x + F.linear(F.silu(F.linear(h, gw)) * F.linear(h, uw), dw)
        for (cache, t) in batch:
            cache.length += len(t)
            cache.tokens += t
        x = ops.rms_norm(x, self.norm, eps)
        if not all_logits:
            x = x[torch.tensor([s0 + T - 1 for s0, T in spans])]
        return F.linear(x, self.lm_head)

    def rope(self, layer: int, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        """q or k rotation of one layer (nanoserve/model.py:242-244). A method so that tests can plant a
        mistake in one layer of the oracle."""
        return ops.apply_rope(x, cos, sin)

    def attend(self, layer: int, q: torch.Tensor, ks: torch.Tensor, vs: torch.Tensor, ctx_len: int) -> torch.Tensor:
        """One sequence's attention in one layer (nanoserve/model.py:283-318): q [T, nh, hd] at positions
        ctx_len ..; ks, vs [ctx_len + T, nkv, hd]. One new token: SDPA with GQA and no mask; several: the
        causal-offset mask. Returns [T, nh, hd]."""
        hd = self.cfg.head_dim
        if q.shape[0] == 1:
            qs = q.transpose(0, 1)[None]
            return F.scaled_dot_product_attention(qs, ks.transpose(0, 1)[None], vs.transpose(0, 1)[None],
                                                  scale=hd ** -0.5, enable_gqa=True)[0].transpose(0, 1)
        return ops.causal_offset_attention(q, ks, vs, ctx_len, hd ** -0.5)

    @torch.inference_mode()
    def teacher_forced(self, prompts: list[list[int]], streams: list[list[int]], max_len: int | None = None):
        """Logits of every generated position of `streams` given their own history: step j of stream i is
        computed on prompt i + streams[i][:j], whatever the oracle itself would have chosen before. Prefill
        one prompt per step, then batched one-token steps (streams of unequal length drop out as they end).
        Returns logits[i][j] ([V] each, the oracle's dtype)."""
        max_len = max_len or max(len(p) + len(s) for p, s in zip(prompts, streams))
        caches = [self.new_cache(max_len) for _ in prompts]
        out: list[list[torch.Tensor]] = [[] for _ in prompts]
        for i, p in enumerate(prompts):
            if streams[i]:
                out[i].append(self.step([(caches[i], list(p))])[0])
        for j in range(1, max(len(s) for s in streams)):
            live = [i for i, s in enumerate(streams) if len(s) > j]
            lg = self.step([(caches[i], [streams[i][j - 1]]) for i in live])
            for r, i in enumerate(live):
                out[i].append(lg[r])
        return out

    def generate_greedy(self, prompts: list[list[int]], n_new: int, max_len: int | None = None,
                        return_logits: bool = False):
        """Prefill every prompt (one step each), then n_new - 1 batched greedy decode steps: the first token
        comes from the prefill logits. Returns the generated tokens per prompt (and the logits of every
        step if asked)."""
        max_len = max_len or max(len(p) for p in prompts) + n_new
        caches = [self.new_cache(max_len) for _ in prompts]
        outs: list[list[int]] = [[] for _ in prompts]
        all_logits = [[] for _ in prompts]
        for i, p in enumerate(prompts):
            lg = self.step([(caches[i], list(p))])[0]
            all_logits[i].append(lg)
            outs[i].append(int(lg.argmax()))
        for _ in range(n_new - 1):
            lg = self.step([(c, [o[-1]]) for c, o in zip(caches, outs)])
            for i in range(len(prompts)):
                all_logits[i].append(lg[i])
                outs[i].append(int(lg[i].argmax()))
        return (outs, all_logits) if return_logits else outs

"""Graph-captured decode of a patched Llama / Qwen2 model over a Quest cache.

After the prompt went through the ``mp_headinfer``-patched model (which fills
the cache's slab and page metadata), ``GraphDecoder`` runs every decode token
as one replay of a single captured graph: the embedding row of the current
token, then per layer the RMSNorm, the q/k/v projections, RoPE at the
device-resident position, the sparse path (ragged Quest selection, page-tile
attention with the decode token's append fused in, the page-metadata update
of the appended row), the output projection and the MLP, then the final norm
and the LM head, and the next token (greedy, or a fixed id as the reference
runner decodes, run_ruler_partial_h2d_tpot_case_v1.py:1302-1322).

Nothing in the graph depends on a host-side length: the token id, the
position and the cache length live in device memory and advance at the end
of the graph, and the ragged kernels derive each group's window, candidate
pages and decode row from the length.  The per-layer arithmetic is the HF
modules' own (same ops, same operand shapes), so logits follow the eager
patched model.  Quest selection with an absolute budget (``budget_pages``),
16-row pages, head_dim 128 and 16-bit K/V only (the page-tile kernel); the
cache must be built with ``update_metadata_on_decode=True`` so pages
completed during decode are scored.  While the decoder runs it owns the
cache; ``sync_cache()`` brings the cache's host-side lengths up to date.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from . import kernels

__all__ = ["GraphDecoder"]


def _rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """LlamaRMSNorm / Qwen2RMSNorm: fp32 variance, scale in the input dtype."""
    dtype = x.dtype
    h = x.to(torch.float32)
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return weight * h.to(dtype)


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


class GraphDecoder:
    """One captured graph per model: ``step()`` decodes one token."""

    def __init__(self, model: torch.nn.Module, cache, *, max_new_tokens: int, fixed_token: Optional[int] = None):
        if not getattr(cache, "update_metadata_on_decode", False):
            raise ValueError("GraphDecoder needs a cache built with update_metadata_on_decode=True")
        if cache.budget_pages is None:
            raise ValueError("GraphDecoder needs an absolute Quest budget (budget_pages)")
        if type(cache).__name__ != "QuestTopKOffloadedCache":
            raise ValueError("GraphDecoder runs Quest selection; use a QuestTopKOffloadedCache")
        inner = model.model
        cfg = model.config
        self.model, self.cache = model, cache
        self.G = cfg.num_key_value_heads
        self.Hq = cfg.num_attention_heads
        self.R = self.Hq // self.G
        self.D = getattr(cfg, "head_dim", None) or cfg.hidden_size // self.Hq
        self.layers = list(inner.layers)
        if cache.block_size != 16 or self.D != 128 or cache.dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("GraphDecoder needs 16-row pages, head_dim 128 and a 16-bit cache")
        if self.R > 8:
            raise ValueError("at most 8 query heads per KV head")
        if cache.geometry.num_entries != len(self.layers) * self.G:
            raise ValueError("cache entries do not match the model's layers x KV heads")
        lengths = set(cache._logical_lengths)
        if len(lengths) != 1 or cache._page_min is None:
            raise ValueError("prefill the cache through the patched model first")
        L0 = lengths.pop()
        if L0 + max_new_tokens + 1 > cache.geometry.max_cache_len:
            raise ValueError("max_new_tokens does not fit the cache")
        dev = cache.device
        self.dev = dev
        self.L0 = L0
        self.steps_done = 0
        self.max_new_tokens = max_new_tokens
        self.fixed_token = fixed_token
        self.P = min(int(cache._page_min.shape[1]), 8192)
        self.k = min(int(cache.budget_pages), self.P)
        self.width = max(1, min(self.P, self.R * self.k))
        # device state: token, position, per-group length
        self.token = torch.full((1,), 1 if fixed_token is None else int(fixed_token), dtype=torch.long, device=dev)
        self.position = torch.full((1,), L0, dtype=torch.long, device=dev)
        self.lengths = torch.full((self.G,), L0, dtype=torch.int32, device=dev)
        # RoPE table for every position the decoder reaches, from the model's own rotary module
        npos = L0 + max_new_tokens + 1
        dummy = torch.zeros((1, 1, self.D), dtype=cache.dtype, device=dev)
        cos, sin = inner.rotary_emb(dummy, torch.arange(npos, device=dev)[None])
        self.cos, self.sin = cos[0].contiguous(), sin[0].contiguous()
        # per-layer buffers
        self.plan = [(torch.zeros((self.G, self.width), dtype=torch.int32, device=dev),
                      torch.zeros((self.G, self.width), dtype=torch.uint8, device=dev),
                      torch.zeros((self.G,), dtype=torch.int32, device=dev)) for _ in self.layers]
        self.attn = [torch.empty((self.G, self.R, self.D), dtype=cache.dtype, device=dev) for _ in self.layers]
        self.logits: Optional[torch.Tensor] = None
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    # ------------------------------------------------------------------ step
    def _body(self) -> None:
        c = self.cache
        G, R, D, Hq = self.G, self.R, self.D, self.Hq
        inner = self.model.model
        h = F.embedding(self.token, inner.embed_tokens.weight)          # [1, hidden]
        cos = self.cos.index_select(0, self.position)                   # [1, D]
        sin = self.sin.index_select(0, self.position)
        for li, layer in enumerate(self.layers):
            attn = layer.self_attn
            x = _rms_norm(h, layer.input_layernorm.weight, layer.input_layernorm.variance_epsilon)
            q = attn.q_proj(x).view(Hq, D)
            k = attn.k_proj(x).view(G, D)
            v = attn.v_proj(x).view(G, D)
            q = (q * cos) + (_rotate_half(q) * sin)
            k = (k * cos) + (_rotate_half(k) * sin)
            qg = q.view(G, R, D).contiguous()
            e0 = li * G
            pp, pm, pc = self.plan[li]
            kernels.quest_select_ragged(qg.float(), c._page_min[e0:e0 + G, :self.P], c._page_max[e0:e0 + G, :self.P],
                                        self.lengths, self.k, sink=c.sink_tokens, recent=c.recent_tokens,
                                        block_size=c.block_size, plan_pages=pp, plan_masks=pm, plan_counts=pc)
            if c.previous_token_resident_cache:
                kernels.decode_attention_pages_resident(qg, c._key_cache[e0:e0 + G], c._value_cache[e0:e0 + G], pp,
                                                        pc, c.resident_pages().view(e0, G), lengths=self.lengths,
                                                        plan_masks=pm, max_pages=self.width, sink=c.sink_tokens,
                                                        recent=c.recent_tokens, block_size=c.block_size, append=True,
                                                        cur_k=k.contiguous(), cur_v=v.contiguous(),
                                                        softmax_scale=float(attn.scaling), out=self.attn[li])
            else:
                kernels.decode_attention_pages_ragged(qg, c._key_cache[e0:e0 + G], c._value_cache[e0:e0 + G], pp,
                                                      pc, self.lengths, plan_masks=pm, max_pages=self.width,
                                                      sink=c.sink_tokens, recent=c.recent_tokens,
                                                      block_size=c.block_size, append=True, cur_k=k.contiguous(),
                                                      cur_v=v.contiguous(), softmax_scale=float(attn.scaling),
                                                      out=self.attn[li])
            kernels.update_page_metadata_ragged(c._key_cache, self.lengths, first_entry=e0, sink=c.sink_tokens,
                                                block_size=c.block_size, page_min=c._page_min, page_max=c._page_max)
            h = h + attn.o_proj(self.attn[li].view(1, Hq * D))
            x = _rms_norm(h, layer.post_attention_layernorm.weight, layer.post_attention_layernorm.variance_epsilon)
            mlp = layer.mlp
            h = h + mlp.down_proj(mlp.act_fn(mlp.gate_proj(x)) * mlp.up_proj(x))
        h = _rms_norm(h, inner.norm.weight, inner.norm.variance_epsilon)
        logits = self.model.lm_head(h)
        if self.logits is None:
            self.logits = torch.empty_like(logits)
        self.logits.copy_(logits)
        if self.fixed_token is None:
            self.token.copy_(logits.argmax(dim=-1))
        self.position.add_(1)
        self.lengths.add_(1)

    def capture(self) -> None:
        """Capture the step graph.  The step runs once eagerly first (its
        token counts as decoded): workspaces and the logits buffer are
        allocated outside the capture."""
        if self.graph is not None:
            return
        self._guard(1)
        with torch.no_grad():
            self._body()
            torch.cuda.synchronize(self.dev)
            self.steps_done += 1
            stream = torch.cuda.Stream(device=self.dev)
            stream.wait_stream(torch.cuda.current_stream(self.dev))
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(stream):
                with torch.cuda.graph(graph, stream=stream):
                    self._body()
            torch.cuda.current_stream(self.dev).wait_stream(stream)
            torch.cuda.synchronize(self.dev)
        self.graph = graph

    def _guard(self, n: int) -> None:
        if self.steps_done + n > self.max_new_tokens:
            raise RuntimeError("GraphDecoder decoded max_new_tokens already")

    def step(self) -> torch.Tensor:
        """Decode one token; returns the logits buffer [1, vocab] (valid until
        the next step)."""
        if self.graph is None:
            self.capture()
            assert self.logits is not None
            return self.logits
        self._guard(1)
        self.graph.replay()
        self.steps_done += 1
        assert self.logits is not None
        return self.logits

    def sync_cache(self) -> None:
        """Advance the cache's host-side lengths over the tokens decoded by
        the graph, so the eager API can take over again."""
        c = self.cache
        n = self.steps_done - getattr(self, "_synced", 0)
        if n <= 0:
            return
        torch.cuda.synchronize(self.dev)
        for e in range(c.geometry.num_entries):
            c._bookkeeping.advance(e, n)
            c._initialized[e] = True
        c._seen_tokens = c._bookkeeping.seen_tokens
        self._synced = self.steps_done

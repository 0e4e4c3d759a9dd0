"""Graph-captured decode of a patched Llama / Qwen2 model over a Quest or a
Twilight cache.

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
pages and decode row from the length.  A layer is 8 launches: the q/k/v
GEMV with the residual add + RMSNorm before it and RoPE after it (q also in
fp32 for the Quest score), the Quest score and top-k, the page-tile
attention (which also appends the decode token and updates the min/max of
a page it completes) and its merge, the output GEMV, the gate/up GEMV with
the residual add + RMSNorm before it and SiLU * up after it, and the down
GEMV (one token, memory-bound, fp32 accumulation).  The residual stream
alternates between two buffers, since every GEMV block normalises the row
itself while block 0 stores the sum.  With fuse=False the norms, RoPE, SiLU
and the metadata update run as launches of their own (13 per layer) -- the
same bits.
Over a Twilight cache the sparse path of a layer is the ragged Quest B0
selection, the INT4 QK, the top-p (with matched budgets, the allocation
and each head's top-allocated rows) and the GQA union, the union attention
with the append and the INT4 + page metadata update of the appended row,
all from the device-side lengths.
The q/k/v and gate/up weights are concatenated once and the HF modules keep
views into them, so the model's own forward (the prefill) uses the same
storage.  The element-wise steps repeat the HF modules' rounding steps; the
GEMV and RMSNorm reduction orders differ from hipBLASLt and torch, so logits
follow the eager patched model to bf16 rounding.  Quest selection needs an
absolute budget (``budget_pages``); both caches need 16-row pages, head_dim
128 and 16-bit K/V, and must be built with ``update_metadata_on_decode=True``
so pages completed during decode are scored.  While the decoder runs it owns the
cache; ``sync_cache()`` brings the cache's host-side lengths up to date.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F

from . import kernels

__all__ = ["GraphDecoder"]


class GraphDecoder:
    """One captured graph per model: ``step()`` decodes one token."""

    def __init__(self, model: torch.nn.Module, cache, *, max_new_tokens: int, fixed_token: Optional[int] = None,
                 fuse: bool = True, dense: bool = False):
        if not getattr(cache, "update_metadata_on_decode", False):
            raise ValueError("GraphDecoder needs a cache built with update_metadata_on_decode=True")
        kind = type(cache).__name__
        if kind == "TwilightMatchedBudgetOffloadedCache":
            # (its resident cache, when active, rides in the fused union attention)
            self.twilight = True
        elif kind == "QuestTopKOffloadedCache":
            self.twilight = False
            if cache.budget_pages is None and not dense:
                raise ValueError("GraphDecoder needs an absolute Quest budget (budget_pages)")
            if dense and cache.previous_token_resident_cache:
                raise ValueError("the dense comparator reads the slab directly (no resident cache)")
        else:
            raise ValueError("GraphDecoder runs a QuestTopKOffloadedCache or a TwilightMatchedBudgetOffloadedCache")
        if dense and self.twilight:
            raise ValueError("the dense comparator runs over a Quest cache")
        # dense: no selection at all -- every whole page between the sink and
        # the recent window is attended through the same page-tile kernel (the
        # plan is every page, ascending), i.e. all rows but the <= bs - 1 rows
        # of the partial page before the recent window
        self.dense = bool(dense)
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
        if self.R > 8 and not (self.twilight and (cache.budget_mode == "dynamic" or self.R <= 64)):
            # the Twilight fused selection and union attention run wider groups
            # as sub-groups of 8 (matched budgets: up to 64 heads sharing one
            # allocation); the Quest page-tile launches take at most 8 heads a group
            raise ValueError("GraphDecoder takes at most 8 query heads per KV head, except over a Twilight cache "
                             "(dynamic budgets, or matched budgets up to 64 heads)")
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
        self.fuse = fuse
        self.P = int(cache._page_min.shape[1])
        if self.twilight:
            # stage 1 keeps B0 pages per head (fewer for a short group), stage 2 top-p over their tokens
            self.k = min(max(1, math.ceil(cache.candidate_token_budget / cache.block_size)), self.P)
        else:
            self.k = self.P if self.dense else min(int(cache.budget_pages), self.P)
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
        # fused projections: one q/k/v and one gate/up weight per layer, the HF modules keep views
        self.wqkv, self.bqkv, self.wgu, self.bgu = [], [], [], []
        with torch.no_grad():
            for layer in self.layers:
                at, mlp = layer.self_attn, layer.mlp
                projs = (at.q_proj, at.k_proj, at.v_proj)
                w = torch.cat([p.weight for p in projs]).contiguous()
                b = torch.cat([p.bias for p in projs]).contiguous() if at.q_proj.bias is not None else None
                o = 0
                for p in projs:
                    n = p.weight.shape[0]
                    p.weight.data = w[o:o + n]
                    if b is not None:
                        p.bias.data = b[o:o + n]
                    o += n
                gu = torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight]).contiguous()
                ni = mlp.gate_proj.weight.shape[0]
                mlp.gate_proj.weight.data = gu[:ni]
                mlp.up_proj.weight.data = gu[ni:]
                bgu = None
                if mlp.gate_proj.bias is not None:
                    bgu = torch.cat([mlp.gate_proj.bias, mlp.up_proj.bias]).contiguous()
                    mlp.gate_proj.bias.data = bgu[:ni]
                    mlp.up_proj.bias.data = bgu[ni:]
                self.wqkv.append(w)
                self.bqkv.append(b)
                self.wgu.append(gu)
                self.bgu.append(bgu)
        self.I = self.wgu[0].shape[0] // 2
        hidden = cfg.hidden_size
        self.x = torch.empty((1, hidden), dtype=cache.dtype, device=dev)
        self.qkv = torch.empty((1, self.wqkv[0].shape[0]), dtype=cache.dtype, device=dev)
        self.o = torch.empty((1, hidden), dtype=cache.dtype, device=dev)
        self.gu = torch.empty((1, self.wgu[0].shape[0]), dtype=cache.dtype, device=dev)
        self.dn = torch.empty((1, hidden), dtype=cache.dtype, device=dev)
        self.vocab = model.lm_head.weight.shape[0]
        self.q32 = torch.empty((self.Hq, self.D), dtype=torch.float32, device=dev)
        self.m = torch.empty((1, self.I), dtype=cache.dtype, device=dev)
        self.hbuf = [torch.empty((1, hidden), dtype=cache.dtype, device=dev) for _ in range(2)]
        # per-layer buffers
        self.plan = [(torch.zeros((self.G, self.width), dtype=torch.int32, device=dev),
                      torch.zeros((self.G, self.width), dtype=torch.uint8, device=dev),
                      torch.zeros((self.G,), dtype=torch.int32, device=dev)) for _ in self.layers]
        self.attn = [torch.empty((self.G, self.R, self.D), dtype=cache.dtype, device=dev) for _ in self.layers]
        # sparse Quest over an HBM or host slab (no resident page cache): each
        # head's selection as a page bitmap, ranked by the attention
        self.use_bits = (not self.twilight and not self.dense and not cache.previous_token_resident_cache
                         and self.P <= 8192 and self.R <= 8)
        if self.use_bits:
            self.bits = torch.zeros((len(self.layers), self.G, self.R, kernels.sel_bits_words(self.P)),
                                    dtype=torch.int32, device=dev)
        if self.dense:
            self.dense_pages = torch.arange(self.width, dtype=torch.int32, device=dev).expand(self.G, -1).contiguous()
            self.dense_masks = torch.full((self.G, self.width), (1 << self.R) - 1, dtype=torch.uint8, device=dev)
            self.dense_counts = torch.zeros((self.G,), dtype=torch.int32, device=dev)
        if self.twilight:
            # stage-2 buffers, reused layer after layer: B0 pages, INT4 logits, union rows
            self.max_length = L0 + max_new_tokens
            n_cand = self.k * cache.block_size
            self.tw_sel = torch.zeros((self.G, self.R, self.k), dtype=torch.int32, device=dev)
            self.tw_logits = torch.zeros((self.G, self.R, n_cand), dtype=torch.float32, device=dev)
            self.tw_rows = torch.zeros((self.G, self.max_length + 1), dtype=torch.int32, device=dev)
            self.tw_counts = torch.zeros((self.G,), dtype=torch.int32, device=dev)
            self.tw_max_rows = min(self.max_length, cache.sink_tokens + self.R * n_cand + cache.recent_tokens)
            # 16-row pages at D = 128, 16-bit K/V, R <= 8: the kept rows as row
            # masks of the B0 union pages, attended page by page
            self.page_rows = (cache.block_size == 16 and self.D == 128 and self.R <= 8
                              and cache.dtype in (torch.float16, torch.bfloat16))
            self.tw_slot_u = torch.zeros((self.G, self.R, self.k), dtype=torch.int32, device=dev)
            self.tw_prows = torch.zeros((self.G, self.width), dtype=torch.int32, device=dev)
            # the fused selection (score + INT4 QK; B0 + top-p per head) into a
            # union record per KV group, read by the union attention; more
            # than 8 query heads per KV head as sub-groups (matched budgets:
            # up to 64 heads, one allocation over all of them)
            self.fused = (cache.block_size == 16 and self.D == 128 and cache.dtype in (torch.float16, torch.bfloat16)
                          and (self.R <= 64 or cache.budget_mode == "dynamic") and self.P <= 8192
                          and n_cand <= 8192)
            if cache.budget_mode == "matched":
                if not self.fused:
                    raise ValueError("GraphDecoder runs matched Twilight budgets through the fused selection "
                                     "(16-row pages, head_dim 128, 16-bit K/V, R <= 64, <= 8192 candidate pages)")
                # the matched target grows with the length while B0 stops at k
                # pages: past that the reference's allocation raises, so refuse
                # a decode that would reach it
                L = self.max_length
                sink_end = min(cache.sink_tokens, L)
                recent_start = max(sink_end, L - max(0, cache.recent_tokens - 1))
                eligible = recent_start - sink_end
                cand = min(eligible // cache.block_size, self.P)
                fixed = min(cand, max(1, math.ceil(cache.matched_budget_fraction * eligible / cache.block_size)))
                if fixed > min(cand, self.k):
                    raise ValueError("matched budget past the B0 candidates before max_new_tokens "
                                     f"({fixed} > {min(cand, self.k)} pages)")
            words = (kernels.union_record_words(self.P) + 3) & ~3
            self.tw_rec = torch.zeros((self.G, words), dtype=torch.int32, device=dev)
            self.tw_desired = torch.zeros((self.G, self.R), dtype=torch.int32, device=dev)
        self.logits: Optional[torch.Tensor] = None
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    # ------------------------------------------------------------------ step
    def _body(self) -> None:
        c = self.cache
        G, R, D, Hq = self.G, self.R, self.D, self.Hq
        inner = self.model.model
        h = F.embedding(self.token, inner.embed_tokens.weight)          # [1, hidden], the residual stream
        x = self.x
        delta: Optional[torch.Tensor] = None
        flip = 0

        def norm_into(norm, weight, bias, out, epilogue, **kw) -> None:
            # fused: h_out = h + delta goes to the buffer h is not in
            nonlocal h, flip
            h_out = None
            if delta is not None:
                h_out = self.hbuf[flip]
                flip ^= 1
            kernels.rms_norm_gemv(h, delta, norm.weight, norm.variance_epsilon, h_out, weight, bias, out,
                                  epilogue=epilogue, **kw)
            if h_out is not None:
                h = h_out

        if self.dense:
            # every whole page between the sink and the recent window, per group
            L = self.lengths
            sink_end = L.clamp(max=c.sink_tokens)
            recent_start = torch.maximum(sink_end, L - max(0, c.recent_tokens - 1))
            self.dense_counts.copy_(((recent_start - sink_end) // c.block_size).clamp(0, self.width))
        for li, layer in enumerate(self.layers):
            attn = layer.self_attn
            norm = layer.input_layernorm
            if self.fuse:
                norm_into(norm, self.wqkv[li], self.bqkv[li], self.qkv, "rope",
                          rope=(Hq, G, self.cos, self.sin, self.position), q32=self.q32)
                qkv = self.qkv[0]
            else:
                kernels.add_rms_norm(h, delta, norm.weight, norm.variance_epsilon, x)
                qkv = kernels.gemv(x, self.wqkv[li], self.bqkv[li], self.qkv)[0]
            q = qkv[:Hq * D].view(Hq, D)
            k = qkv[Hq * D:(Hq + G) * D].view(G, D)
            v = qkv[(Hq + G) * D:].view(G, D)
            if not self.fuse:
                kernels.rope_qk(q, k, self.cos, self.sin, self.position, self.q32)
            qg = q.view(G, R, D)
            e0 = li * G
            pp, pm, pc = self.plan[li]
            if self.twilight:
                self._twilight_attention(li, attn, qg, k, v, pp, pm, pc)
                o = kernels.gemv(self.attn[li].view(1, Hq * D), attn.o_proj.weight, attn.o_proj.bias, self.o)
                norm = layer.post_attention_layernorm
                delta = o
                if self.fuse:
                    norm_into(norm, self.wgu[li], self.bgu[li], self.m, "silu")
                else:
                    kernels.add_rms_norm(h, o, norm.weight, norm.variance_epsilon, x)
                    gu = kernels.gemv(x, self.wgu[li], self.bgu[li], self.gu)
                    kernels.silu_mul(gu, self.m)
                delta = kernels.gemv(self.m, layer.mlp.down_proj.weight, layer.mlp.down_proj.bias, self.dn)
                continue
            if self.use_bits:
                bits = self.bits[li]
                kernels.quest_select_bits(self.q32.view(G, R, D), c._page_min[e0:e0 + G, :self.P],
                                          c._page_max[e0:e0 + G, :self.P], self.k, bits, lengths=self.lengths,
                                          sink=c.sink_tokens, recent=c.recent_tokens, block_size=c.block_size)
                meta = dict(page_min=c._page_min[e0:e0 + G], page_max=c._page_max[e0:e0 + G]) if self.fuse else {}
                kernels.decode_attention_pages_bits(qg, c._key_cache[e0:e0 + G], c._value_cache[e0:e0 + G], bits,
                                                    self.P, max_pages=self.width, sink=c.sink_tokens,
                                                    recent=c.recent_tokens, block_size=c.block_size,
                                                    lengths=self.lengths, append=True, cur_k=k, cur_v=v,
                                                    softmax_scale=float(attn.scaling), out=self.attn[li], **meta)
            elif self.dense:
                pp, pm, pc = self.dense_pages, self.dense_masks, self.dense_counts
                meta = {}
            else:
                kernels.quest_select_ragged(self.q32.view(G, R, D), c._page_min[e0:e0 + G, :self.P],
                                            c._page_max[e0:e0 + G, :self.P], self.lengths, self.k,
                                            sink=c.sink_tokens, recent=c.recent_tokens, block_size=c.block_size,
                                            plan_pages=pp, plan_masks=pm, plan_counts=pc)
                # the attention also appends the decode token and, when it completes a page, that page's min/max
                meta = dict(page_min=c._page_min[e0:e0 + G], page_max=c._page_max[e0:e0 + G]) if self.fuse else {}
            if self.use_bits:
                pass
            elif c.previous_token_resident_cache:
                kernels.decode_attention_pages_resident(qg, c._key_cache[e0:e0 + G], c._value_cache[e0:e0 + G], pp,
                                                        pc, c.resident_pages().view(e0, G), lengths=self.lengths,
                                                        plan_masks=pm, max_pages=self.width, sink=c.sink_tokens,
                                                        recent=c.recent_tokens, block_size=c.block_size, append=True,
                                                        cur_k=k, cur_v=v, softmax_scale=float(attn.scaling),
                                                        out=self.attn[li], **meta)
            else:
                kernels.decode_attention_pages_ragged(qg, c._key_cache[e0:e0 + G], c._value_cache[e0:e0 + G], pp,
                                                      pc, self.lengths, plan_masks=pm, max_pages=self.width,
                                                      sink=c.sink_tokens, recent=c.recent_tokens,
                                                      block_size=c.block_size, append=True, cur_k=k, cur_v=v,
                                                      softmax_scale=float(attn.scaling), out=self.attn[li], **meta)
            if not self.fuse and not self.dense:
                kernels.update_page_metadata_ragged(c._key_cache, self.lengths, first_entry=e0, sink=c.sink_tokens,
                                                    block_size=c.block_size, page_min=c._page_min,
                                                    page_max=c._page_max)
            o = kernels.gemv(self.attn[li].view(1, Hq * D), attn.o_proj.weight, attn.o_proj.bias, self.o)
            norm = layer.post_attention_layernorm
            delta = o
            if self.fuse:
                norm_into(norm, self.wgu[li], self.bgu[li], self.m, "silu")
            else:
                kernels.add_rms_norm(h, o, norm.weight, norm.variance_epsilon, x)
                gu = kernels.gemv(x, self.wgu[li], self.bgu[li], self.gu)
                kernels.silu_mul(gu, self.m)
            delta = kernels.gemv(self.m, layer.mlp.down_proj.weight, layer.mlp.down_proj.bias, self.dn)
        if self.logits is None:
            self.logits = torch.empty((1, self.vocab), dtype=self.cache.dtype, device=self.dev)
        if self.fuse:
            norm_into(inner.norm, self.model.lm_head.weight, self.model.lm_head.bias, self.logits, "plain")
            logits = self.logits
        else:
            kernels.add_rms_norm(h, delta, inner.norm.weight, inner.norm.variance_epsilon, x)
            logits = kernels.gemv(x, self.model.lm_head.weight, self.model.lm_head.bias, self.logits)
        if self.fixed_token is None:
            self.token.copy_(logits.argmax(dim=-1))
        self.position.add_(1)
        self.lengths.add_(1)

    def _twilight_attention(self, li: int, attn, qg, k, v, pp, pm, pc) -> None:
        """Twilight stages 1-2 (Quest B0, INT4 QK, top-p + GQA union) and the
        union attention with the append, then the INT4 row and page metadata
        of the appended row, all from the device-side lengths."""
        c = self.cache
        G, R, D = self.G, self.R, self.D
        e0 = li * G
        q32 = self.q32.view(G, R, D)
        if self.fused:
            kernels.twilight_select_fused(q32, c._page_min[e0:e0 + G, :self.P], c._page_max[e0:e0 + G, :self.P],
                                          c._packed[e0:e0 + G], c._qscale[e0:e0 + G], c._qmin[e0:e0 + G], self.k,
                                          self.tw_rec, top_p=c.top_p, sink=c.sink_tokens, recent=c.recent_tokens,
                                          block_size=c.block_size, length=self.max_length, lengths=self.lengths,
                                          desired=self.tw_desired, budget_mode=c.budget_mode,
                                          sel_pages=self.tw_sel if c.budget_mode == "matched" else None,
                                          matched_fraction=c.matched_budget_fraction)
            # the attention also appends the decode token and (fused) its INT4 row and page metadata
            meta = dict(page_min=c._page_min[e0:e0 + G], page_max=c._page_max[e0:e0 + G],
                        packed=c._packed[e0:e0 + G], scale=c._qscale[e0:e0 + G],
                        minimum=c._qmin[e0:e0 + G]) if self.fuse else {}
            resident = c.resident_pages().view(e0, G) if c._resident_active else None
            kernels.decode_attention_union(qg, c._key_cache[e0:e0 + G], c._value_cache[e0:e0 + G], self.tw_rec,
                                           self.P, max_pages=self.width, sink=c.sink_tokens,
                                           recent=c.recent_tokens, block_size=c.block_size, lengths=self.lengths,
                                           append=True, cur_k=k, cur_v=v, softmax_scale=float(attn.scaling),
                                           out=self.attn[li], resident=resident, **meta)
            if not self.fuse:
                kernels.update_page_metadata_ragged(c._key_cache, self.lengths, first_entry=e0, sink=c.sink_tokens,
                                                    block_size=c.block_size, page_min=c._page_min,
                                                    page_max=c._page_max, packed=c._packed, scale=c._qscale,
                                                    minimum=c._qmin)
            return
        kernels.quest_select_ragged(q32, c._page_min[e0:e0 + G, :self.P], c._page_max[e0:e0 + G, :self.P],
                                    self.lengths, self.k, sink=c.sink_tokens, recent=c.recent_tokens,
                                    block_size=c.block_size, sel_pages=self.tw_sel, plan_pages=pp, plan_masks=pm,
                                    plan_counts=pc)
        if self.page_rows:
            kernels.twilight_qk(q32, c._packed[e0:e0 + G], c._qscale[e0:e0 + G], c._qmin[e0:e0 + G], pp, pm, pc,
                                self.k, sink=c.sink_tokens, block_size=c.block_size, out=self.tw_logits,
                                slot_u=self.tw_slot_u, page_rows=self.tw_prows)
            kernels.twilight_select_pages(self.tw_logits, self.tw_sel, self.tw_slot_u, self.tw_prows, top_p=c.top_p,
                                          sink=c.sink_tokens, recent=c.recent_tokens, block_size=c.block_size,
                                          length=self.max_length, lengths=self.lengths, page_capacity=self.P)
            # the attention also appends the decode token and (fused) its INT4 row and page metadata
            meta = dict(page_min=c._page_min[e0:e0 + G], page_max=c._page_max[e0:e0 + G],
                        packed=c._packed[e0:e0 + G], scale=c._qscale[e0:e0 + G],
                        minimum=c._qmin[e0:e0 + G]) if self.fuse else {}
            kernels.decode_attention_page_rows(qg, c._key_cache[e0:e0 + G], c._value_cache[e0:e0 + G], pp, pc,
                                               self.tw_prows, max_pages=self.width, sink=c.sink_tokens,
                                               recent=c.recent_tokens, block_size=c.block_size, lengths=self.lengths,
                                               append=True, cur_k=k, cur_v=v, softmax_scale=float(attn.scaling),
                                               out=self.attn[li], **meta)
        else:
            kernels.twilight_qk(q32, c._packed[e0:e0 + G], c._qscale[e0:e0 + G], c._qmin[e0:e0 + G], pp, pm, pc,
                                self.k, sink=c.sink_tokens, block_size=c.block_size, out=self.tw_logits)
            self._twilight_rows_attention(li, attn, qg, k, v)
        if not self.fuse:
            kernels.update_page_metadata_ragged(c._key_cache, self.lengths, first_entry=e0, sink=c.sink_tokens,
                                                block_size=c.block_size, page_min=c._page_min,
                                                page_max=c._page_max, packed=c._packed, scale=c._qscale,
                                                minimum=c._qmin)

    def _twilight_rows_attention(self, li: int, attn, qg, k, v) -> None:
        """Top-p + the GQA union as a row list, then the rows-mode attention
        with the append (shapes the page-row path does not take)."""
        c = self.cache
        G = self.G
        e0 = li * G
        kernels.twilight_select_ragged(self.tw_logits, self.tw_sel, self.lengths, top_p=c.top_p, rows=self.tw_rows,
                                       row_counts=self.tw_counts, max_length=self.max_length,
                                       page_capacity=self.P, sink=c.sink_tokens, recent=c.recent_tokens,
                                       block_size=c.block_size)
        # the attention also appends the decode token and (fused) updates its INT4 row and page metadata
        meta = dict(sink=c.sink_tokens, page_min=c._page_min[e0:e0 + G], page_max=c._page_max[e0:e0 + G],
                    packed=c._packed[e0:e0 + G], scale=c._qscale[e0:e0 + G], minimum=c._qmin[e0:e0 + G])
        kernels.decode_attention_rows(qg, c._key_cache[e0:e0 + G], c._value_cache[e0:e0 + G], self.tw_rows,
                                      self.tw_counts, self.tw_max_rows, cur_k=k, cur_v=v,
                                      softmax_scale=float(attn.scaling), out=self.attn[li],
                                      append_position=self.lengths, metadata=meta if self.fuse else None)

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

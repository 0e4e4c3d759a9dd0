"""Torch-CPU port of the reference's sparse-decode layer step -- TEST
INFRASTRUCTURE ONLY (the ``cpu_baseline`` leg of bench.py and a cross-check in
tests).  Nothing in the product imports it.

It replays, on host tensors, the op sequence the reference runs for one
decoder layer of the Quest per-head path:

* score:  ``where(q > 0, page_max, page_min).float() * q`` summed over D
  (quest_offload_cache.py:362-372);
* select: ``topk(sorted=False)`` then ascending sort (:373-374);
* expand: sink ++ ``sink + page*bs + arange(bs)`` ++ recent (:403-490);
* gather: ``index_select`` of each query head's positions from the entry's
  K/V (:576-587);
* attention: SDPA math over those rows plus the decode token, one query head
  at a time (decode_reference_attention.py:18-69, is_causal False at q_len 1).
"""

from __future__ import annotations

import math
import time
from typing import Optional

import torch
import torch.nn.functional as F


def quest_layer_step(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, page_min: torch.Tensor,
                     page_max: torch.Tensor, cur_k: torch.Tensor, cur_v: torch.Tensor, *, length: int, budget: int,
                     sink: int, recent: int, block_size: int,
                     phases: Optional[dict] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """One layer: q [G,R,D]; k_cache/v_cache [G,>=L,D]; page_min/page_max
    [G,P,D] (the P scored pages); cur_k/cur_v [G,D].  phases (optional)
    accumulates seconds per phase: "score_select", "gather", "attention".

    Returns (out [G,R,D] in q's dtype, selected pages [G,R,budget] int64)."""
    clock = time.perf_counter
    t0 = clock()
    G, R, D = q.shape
    sink_end = min(sink, length)
    recent_start = max(sink_end, length - max(0, recent - 1))
    qf = q.reshape(G * R, D).float()
    pmin = page_min.repeat_interleave(R, dim=0)
    pmax = page_max.repeat_interleave(R, dim=0)
    extrema = torch.where(qf.unsqueeze(1) > 0, pmax, pmin)
    scores = (extrema.float() * qf.unsqueeze(1)).sum(dim=-1)
    chosen = torch.topk(scores, k=budget, dim=-1, largest=True, sorted=False).indices.sort(dim=-1).values
    t_sel = clock() - t0
    t_gather = t_attn = 0.0
    sink_idx = torch.arange(sink_end, dtype=torch.long)
    recent_idx = torch.arange(recent_start, length, dtype=torch.long)
    offsets = torch.arange(block_size, dtype=torch.long)
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(D)
    for g in range(G):
        for r in range(R):
            pages = chosen[g * R + r]
            blocks = (sink + pages.unsqueeze(1) * block_size + offsets.unsqueeze(0)).reshape(-1)
            t1 = clock()
            pos = torch.cat((sink_idx, blocks, recent_idx))
            keys = torch.cat((k_cache[g].index_select(0, pos), cur_k[g : g + 1]))
            vals = torch.cat((v_cache[g].index_select(0, pos), cur_v[g : g + 1]))
            t2 = clock()
            o = F.scaled_dot_product_attention(q[g, r].view(1, 1, 1, D).float(), keys.view(1, 1, -1, D).float(),
                                               vals.view(1, 1, -1, D).float(), is_causal=False, scale=scale)
            out[g, r] = o.view(D).to(q.dtype)
            t_gather += t2 - t1
            t_attn += clock() - t2
    if phases is not None:
        for name, t in (("score_select", t_sel), ("gather", t_gather), ("attention", t_attn)):
            phases[name] = phases.get(name, 0.0) + t
    return out, chosen.view(G, R, budget)


def twilight_layer_step(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, page_min: torch.Tensor,
                        page_max: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, minimum: torch.Tensor,
                        cur_k: torch.Tensor, cur_v: torch.Tensor, *, length: int, b0_pages: int, top_p: float,
                        sink: int, recent: int, block_size: int, budget_mode: str = "dynamic",
                        fixed_pages: int = 0, phases: Optional[dict] = None) -> tuple[torch.Tensor, list]:
    """One layer of the Twilight path on host tensors, in the reference's op
    order (twilight_offload_cache.py:1128-1614): Quest B0 pages, candidate
    expansion, INT4 dequantize + fp32 matmul / sqrt(D), argsort + softmax +
    cumsum + searchsorted top-p, with matched budgets the largest-remainder
    allocation towards fixed_pages x block_size x R (:1346-1354, :50-86),
    the per-group token union, then index_select and SDPA over the union plus
    the decode token.

    q [G,R,D]; k_cache/v_cache [G,>=L,D]; page metadata [G,P,D]; packed
    [G,T,D/2] u8, scale/minimum [G,T]; cur_k/cur_v [G,D].  phases (optional)
    accumulates seconds per phase: "score_select" (Quest B0), "int4_qk",
    "top_p" (with the allocation), "union", "gather", "attention".  Returns
    (out [G,R,D], the union of each group as an ascending int64 tensor)."""
    from .oracle import matched_budget_counts

    clock = time.perf_counter
    t = {name: 0.0 for name in ("score_select", "int4_qk", "top_p", "union", "gather", "attention")}
    t0 = clock()
    G, R, D = q.shape
    sink_end = min(sink, length)
    recent_start = max(sink_end, length - max(0, recent - 1))
    qf = q.float()
    extrema = torch.where(qf.reshape(G * R, 1, D) > 0, page_max.repeat_interleave(R, 0),
                          page_min.repeat_interleave(R, 0))
    scores = (extrema.float() * qf.reshape(G * R, 1, D)).sum(dim=-1)
    pages = torch.topk(scores, k=b0_pages, dim=-1, sorted=False).indices.view(G, R, b0_pages)
    offsets = torch.arange(block_size)
    cand = (sink + pages.unsqueeze(-1) * block_size + offsets).reshape(G, R, -1)   # [G,R,N]
    t["score_select"] += clock() - t0
    out = torch.empty_like(q)
    unions = []
    scale_qk = 1.0 / math.sqrt(D)
    threshold = torch.tensor(top_p)
    for g in range(G):
        t1 = clock()
        low = (packed[g] & 0x0F)
        high = (packed[g] >> 4) & 0x0F
        logits = []
        for r in range(R):
            pos = cand[g, r]
            codes = torch.stack((low[pos], high[pos]), dim=-1).flatten(-2).float()
            k_hat = codes * scale[g, pos].float().unsqueeze(-1) + minimum[g, pos].float().unsqueeze(-1)
            logits.append((k_hat @ qf[g, r]) * scale_qk)
        t2 = clock()
        orders, desired = [], []
        for r in range(R):
            order = torch.argsort(logits[r], descending=True)
            cum = torch.cumsum(torch.softmax(logits[r][order], dim=0), dim=0)
            desired.append(min(int(torch.searchsorted(cum, threshold, right=False)) + 1, order.numel()))
            orders.append(order)
        if budget_mode == "matched":
            n = cand.shape[2]
            allocated = matched_budget_counts(desired, fixed_pages * block_size * R, [n] * R)
        else:
            allocated = desired
        t3 = clock()
        selected = [torch.arange(sink_end), torch.arange(recent_start, length)]
        selected += [cand[g, r][orders[r][:allocated[r]]] for r in range(R)]
        union = torch.unique(torch.cat(selected), sorted=True)
        t4 = clock()
        keys = torch.cat((k_cache[g].index_select(0, union), cur_k[g:g + 1])).float()
        vals = torch.cat((v_cache[g].index_select(0, union), cur_v[g:g + 1])).float()
        t5 = clock()
        o = F.scaled_dot_product_attention(qf[g].view(1, R, 1, D), keys.view(1, 1, -1, D).expand(1, R, -1, D),
                                           vals.view(1, 1, -1, D).expand(1, R, -1, D), is_causal=False,
                                           scale=scale_qk)
        out[g] = o.view(R, D).to(q.dtype)
        t6 = clock()
        t["int4_qk"] += t2 - t1
        t["top_p"] += t3 - t2
        t["union"] += t4 - t3
        t["gather"] += t5 - t4
        t["attention"] += t6 - t5
        unions.append(union)
    if phases is not None:
        for name, v in t.items():
            phases[name] = phases.get(name, 0.0) + v
    return out, unions

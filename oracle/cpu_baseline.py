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

import torch
import torch.nn.functional as F


def quest_layer_step(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, page_min: torch.Tensor,
                     page_max: torch.Tensor, cur_k: torch.Tensor, cur_v: torch.Tensor, *, length: int, budget: int,
                     sink: int, recent: int, block_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """One layer: q [G,R,D]; k_cache/v_cache [G,>=L,D]; page_min/page_max
    [G,P,D] (the P scored pages); cur_k/cur_v [G,D].

    Returns (out [G,R,D] in q's dtype, selected pages [G,R,budget] int64)."""
    G, R, D = q.shape
    sink_end = min(sink, length)
    recent_start = max(sink_end, length - max(0, recent - 1))
    qf = q.reshape(G * R, D).float()
    pmin = page_min.repeat_interleave(R, dim=0)
    pmax = page_max.repeat_interleave(R, dim=0)
    extrema = torch.where(qf.unsqueeze(1) > 0, pmax, pmin)
    scores = (extrema.float() * qf.unsqueeze(1)).sum(dim=-1)
    chosen = torch.topk(scores, k=budget, dim=-1, largest=True, sorted=False).indices.sort(dim=-1).values
    sink_idx = torch.arange(sink_end, dtype=torch.long)
    recent_idx = torch.arange(recent_start, length, dtype=torch.long)
    offsets = torch.arange(block_size, dtype=torch.long)
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(D)
    for g in range(G):
        for r in range(R):
            pages = chosen[g * R + r]
            blocks = (sink + pages.unsqueeze(1) * block_size + offsets.unsqueeze(0)).reshape(-1)
            pos = torch.cat((sink_idx, blocks, recent_idx))
            keys = torch.cat((k_cache[g].index_select(0, pos), cur_k[g : g + 1]))
            vals = torch.cat((v_cache[g].index_select(0, pos), cur_v[g : g + 1]))
            o = F.scaled_dot_product_attention(q[g, r].view(1, 1, 1, D).float(), keys.view(1, 1, -1, D).float(),
                                               vals.view(1, 1, -1, D).float(), is_causal=False, scale=scale)
            out[g, r] = o.view(D).to(q.dtype)
    return out, chosen.view(G, R, budget)

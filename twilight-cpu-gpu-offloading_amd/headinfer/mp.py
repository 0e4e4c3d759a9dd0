"""Model integration of the decode path: the attention hook and the model patch.

_flash_attention_varlen_forward keeps the signature of the reference's
patchable wrapper (mp.py:21-52), which the GQA-group, layer-flat and
per-head decode branches call with G sequences of one query token each.
Here it runs the gfx950 split-K decode attention (tw_decode_attention in
varlen mode): softmax(q.k / sqrt(D)) v over every key of the sequence (with
q_len 1, causal attention sees all keys), fp32 accumulation, output in the
input dtype.  Only decode calls (max_seqlen_q == 1) are served.

mp_headinfer(model) is the reference's patch (mp.py:601-626) for the
transformers attention API of this image (transformers 5.x has no
LlamaFlashAttention2 class to patch): every Llama / Qwen2 attention module
gets the head-wise forward below, its KV heads become cache entries
layer * G + g (mp.py:606-613), and the model's attention implementation is
switched to one that creates no attention masks.  Prefill writes each KV
head's keys and values into the cache (which builds the page metadata) and
runs dense causal attention, as the reference does (mp.py:475-482).  Decode
calls the cache's sparse path for the whole layer:

* ``decode_layer`` (Quest or Twilight selection, union, split-K attention
  over the slab, append) when the cache has no reference execution flag set;
* ``prepare_layer_selection`` + ``update_layer_gqa_group_ragged`` +
  ``_flash_attention_varlen_forward`` when ``gqa_groupwise_execution`` is set
  (the branch at mp.py:239-279);
* ``prepare_layer_selection`` + ``update_layer_flat_ragged`` + the varlen hook
  over per-query-head segments when ``layer_flat_ragged_execution`` is set
  (mp.py:283-321);
* per-entry ``update`` and attention over each head's packed rows otherwise
  (the per-head branch, mp.py:424-452).
"""

from __future__ import annotations

import types
from typing import Any, Optional

import torch

from . import kernels

__all__ = ["_flash_attention_varlen_forward", "mp_headinfer", "LlamaAttention_fast_forward",
           "Qwen2Attention_fast_forward", "ATTN_IMPLEMENTATION"]

ATTN_IMPLEMENTATION = "headinfer"


def _flash_attention_varlen_forward(
    query_states: torch.Tensor,
    key_states: torch.Tensor,
    value_states: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    *,
    dropout: float,
    is_causal: bool,
    sliding_window: Optional[int] = None,
    softmax_scale: Optional[float] = None,
) -> torch.Tensor:
    """query_states [B, Hq, D] (one token per sequence), key/value_states
    [total_k, Hk, D], cu_seqlens_k [B+1] int32 -> [B, Hq, D].  A
    sliding_window w shorter than max_seqlen_k keeps the last w + 1 keys
    (flash-attn window_size=(w, w))."""
    if int(max_seqlen_q) != 1:
        raise NotImplementedError("only decode attention (one query token per sequence) is implemented")
    if dropout:
        raise ValueError("decode attention takes no dropout")
    del is_causal  # one query token aligned to the end of its keys sees all of them
    B = query_states.shape[0]
    if cu_seqlens_q.shape != (B + 1,):
        raise ValueError("cu_seqlens_q must be [B + 1]")
    window = sliding_window if sliding_window is not None and max_seqlen_k > sliding_window else -1
    return kernels.decode_attention_varlen(query_states.contiguous(), key_states.contiguous(),
                                           value_states.contiguous(), cu_seqlens_k, int(max_seqlen_k),
                                           softmax_scale=softmax_scale, window_left=int(window))


# ------------------------------------------------------------------ prefill
def _prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                       chunk: int = 1024) -> torch.Tensor:
    """Dense causal attention of a prompt, q [1, Hq, S, D], k/v [1, G, S, D]
    -> [1, S, Hq*D].  Query chunks keep the score tile bounded; the key
    operand is materialised transposed and contiguous, scores and softmax in
    fp32, p.v with p in the input dtype."""
    _, Hq, S, D = q.shape
    G = k.shape[1]
    R = Hq // G
    qg = q[0].reshape(G, R, S, D)
    kt = k[0].transpose(1, 2).contiguous()           # [G, D, S]
    vv = v[0].contiguous()                           # [G, S, D]
    out = torch.empty((S, G, R, D), dtype=q.dtype, device=q.device)
    pos = torch.arange(S, device=q.device)
    for s0 in range(0, S, chunk):
        s1 = min(S, s0 + chunk)
        qc = qg[:, :, s0:s1].reshape(G, R * (s1 - s0), D).contiguous()
        sc = torch.matmul(qc, kt[:, :, :s1].contiguous()).float().view(G, R, s1 - s0, s1) * scale
        future = pos[None, :s1] > pos[s0:s1, None]
        sc.masked_fill_(future, float("-inf"))
        p = torch.softmax(sc, dim=-1).to(q.dtype).view(G, R * (s1 - s0), s1)
        o = torch.matmul(p, vv[:, :s1].contiguous()).view(G, R, s1 - s0, D)
        out[s0:s1] = o.permute(2, 0, 1, 3)
    return out.view(1, S, Hq * D)


def _head_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lengths, scale: float) -> torch.Tensor:
    """Per-entry packs [1, R, Tmax, D] with per-head valid lengths -> [R, D]
    through the varlen kernel (one sequence per head)."""
    R, D = q.shape[1], q.shape[-1]
    ks = torch.cat([k[0, r, :n] for r, n in enumerate(lengths)]).unsqueeze(1)
    vs = torch.cat([v[0, r, :n] for r, n in enumerate(lengths)]).unsqueeze(1)
    cu = torch.tensor([0, *torch.tensor(lengths).cumsum(0).tolist()], dtype=torch.int32, device=q.device)
    return _flash_attention_varlen_forward(q[0, :, 0].reshape(R, 1, D), ks, vs,
                                           torch.arange(R + 1, dtype=torch.int32, device=q.device), cu, 1,
                                           max(lengths), dropout=0.0, is_causal=True,
                                           softmax_scale=scale).reshape(R, D)


# ------------------------------------------------------------------- decode
def _is_headinfer_cache(cache: Any) -> bool:
    return cache is not None and hasattr(cache, "decode_layer") and hasattr(cache, "geometry")


def _decode(self, cache, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """One decode token of one layer through the cache: q [1, Hq, 1, D],
    k/v [1, G, 1, D] (post-RoPE) -> [1, 1, Hq*D]."""
    G = k.shape[1]
    Hq, D = q.shape[1], q.shape[-1]
    R = Hq // G
    e0 = self._headinfer_entry0
    entries = list(range(e0, e0 + G))
    scale = float(self.scaling)
    groupwise = bool(getattr(cache, "gqa_groupwise_execution", False))
    flat = bool(getattr(cache, "layer_flat_ragged_execution", False))
    per_head_ref = bool(getattr(cache, "per_head_varlen_attention_reference", False))
    if not (groupwise or flat or per_head_ref):
        out = cache.decode_layer(queries=q[0, :, 0].reshape(G, R, D).contiguous(),
                                 key_states=k[0, :, 0].contiguous(), value_states=v[0, :, 0].contiguous(),
                                 entries=entries, softmax_scale=scale)
        return out.reshape(1, 1, Hq * D)
    queries = [q[:, g * R:(g + 1) * R] for g in range(G)]
    keys = [k[:, g:g + 1] for g in range(G)]
    values = [v[:, g:g + 1] for g in range(G)]
    if groupwise or flat:
        cache.prepare_layer_selection(entries=entries, queries=queries)
    if groupwise:
        K, V, cu_k, max_k, _ = cache.update_layer_gqa_group_ragged(key_states=keys, value_states=values,
                                                                   queries=queries, entries=entries)
        out = _flash_attention_varlen_forward(q[0, :, 0].reshape(G, R, D), K, V,
                                              torch.arange(G + 1, dtype=torch.int32, device=q.device), cu_k, 1,
                                              max_k, dropout=0.0, is_causal=True, softmax_scale=scale)
        return out.reshape(1, 1, Hq * D)
    if flat:
        K, V, cu_k, max_k, _ = cache.update_layer_flat_ragged(key_states=keys, value_states=values, queries=queries,
                                                              entries=entries)
        out = _flash_attention_varlen_forward(q[0, :, 0].reshape(Hq, 1, D), K, V,
                                              torch.arange(Hq + 1, dtype=torch.int32, device=q.device), cu_k, 1,
                                              max_k, dropout=0.0, is_causal=True, softmax_scale=scale)
        return out.reshape(1, 1, Hq * D)
    outs = []
    for g, entry in enumerate(entries):
        kp, vp = cache.update(keys[g], values[g], entry, {"query_states": queries[g]})
        lengths = cache.get_last_query_head_lengths(entry)
        outs.append(_head_attention(queries[g], kp, vp, lengths, scale))
    return torch.cat(outs).reshape(1, 1, Hq * D)


def _fast_forward(self, hidden_states: torch.Tensor, position_embeddings=None, attention_mask=None,
                  past_key_values=None, **kwargs):
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    bsz, q_len, _ = hidden_states.shape
    if bsz != 1:
        raise ValueError("the head-wise offload path is batch-1 (slab_cache.py:5)")
    hidden_shape = (bsz, q_len, -1, self.head_dim)
    q = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    k = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    cos, sin = position_embeddings
    q, k = apply_rotary_pos_emb(q, k, cos, sin)
    cache = past_key_values
    if not _is_headinfer_cache(cache):
        raise ValueError("a headinfer-patched model needs a QuestTopKOffloadedCache / "
                         "TwilightMatchedBudgetOffloadedCache as past_key_values")
    if q_len > 1:
        G = k.shape[1]
        for g in range(G):
            cache.update(k[:, g:g + 1].contiguous(), v[:, g:g + 1].contiguous(), self._headinfer_entry0 + g)
        attn = _prefill_attention(q, k, v, float(self.scaling))
    else:
        attn = _decode(self, cache, q.contiguous(), k.contiguous(), v.contiguous())
    return self.o_proj(attn), None


LlamaAttention_fast_forward = _fast_forward
Qwen2Attention_fast_forward = _fast_forward


def _no_mask_attention(module, query, key, value, attention_mask, **kwargs):  # pragma: no cover - never called
    raise RuntimeError("headinfer attention runs inside the patched attention forward")


def mp_headinfer(model: torch.nn.Module) -> torch.nn.Module:
    """Patch a Llama / Qwen2 causal LM for the head-wise sparse decode path
    (mp.py:601-626): each attention module's KV heads become cache entries
    layer * num_key_value_heads + g.  Returns the model."""
    from transformers import AttentionInterface

    inner = getattr(model, "model", model)
    layers = getattr(inner, "layers", None)
    if layers is None:
        raise ValueError("expected a decoder-only model with model.layers")
    kinds = {type(model).__name__}
    if not any(name.startswith(("Llama", "Qwen2")) for name in kinds):
        raise ValueError(f"unsupported model {type(model).__name__}: Llama and Qwen2 are patched")
    AttentionInterface.register(ATTN_IMPLEMENTATION, _no_mask_attention)
    entry = 0
    for layer in layers:
        attn = layer.self_attn
        G = attn.config.num_key_value_heads
        Hq = attn.config.num_attention_heads
        if Hq % G:
            raise ValueError("query heads must be a multiple of KV heads")
        attn._headinfer_entry0 = entry
        attn.forward = types.MethodType(_fast_forward, attn)
        entry += G
    config = model.config
    config._attn_implementation = ATTN_IMPLEMENTATION
    for sub in ("text_config",):
        if hasattr(config, sub):
            getattr(config, sub)._attn_implementation = ATTN_IMPLEMENTATION
    model._headinfer_entries = entry
    return model

"""Attention hook of the decode paths.

_flash_attention_varlen_forward keeps the signature of the reference's
patchable wrapper (mp.py:21-52), which the GQA-group, layer-flat and
per-head decode branches call with G sequences of one query token each.
Here it runs the gfx950 split-K decode attention (tw_decode_attention in
varlen mode): softmax(q.k / sqrt(D)) v over every key of the sequence (with
q_len 1, causal attention sees all keys), fp32 accumulation, output in the
input dtype.  Only decode calls (max_seqlen_q == 1) are served; prefill
attention is not part of this library.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import kernels

__all__ = ["_flash_attention_varlen_forward"]


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
                                           window_left=int(window))

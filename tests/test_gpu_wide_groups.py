"""More than 8 query heads per KV head (e.g. 16 for a 64-query / 4-KV-head
model) through the caches' call surface.  The reference has no limit on the
query heads per KV head (quest_offload_cache.py:26-60); the kernels take at
most 8 heads per launch, so the Python layer runs wider groups as sub-groups
of at most 8 heads.  Checked against the oracle exactly as the R <= 8 cache
tests are: selections bit-exact, gathered rows bit-exact, attention within
2e-3 abs + 1e-2 rel of float64."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from helpers import TORCH_DT
from test_gpu_cache import H, _close, _Model, _quest_positions, _same, _say, _twilight_cache, _twilight_expected  # noqa: F401

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("R", [12, 16])
def test_quest_decode_layer_wide_group(H, dev, R):
    G, D, T, sink, recent, bs = 2, 128, 1500, 64, 64, 16
    _say(f"[wide quest decode_layer] R={R}")
    cache = H["quest"].QuestTopKOffloadedCache(num_cache_entries=G, max_cache_len=T + 2, head_dim=D,
                                               num_query_heads_per_kv=R, dtype=torch.float16, device=dev,
                                               sink_tokens=sink, recent_tokens=recent, block_size=bs,
                                               budget_pages=8, kv_residency="hbm")
    model = _Model(G, T, D, "f16", seed=101)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(102)
    for step in range(2):
        q = torch.randn(G, R, D, generator=g).to(torch.float16)
        new = [model.new_token(D) for _ in range(G)]
        nk = torch.stack([k for k, _ in new])
        nv = torch.stack([v for _, v in new])
        out = cache.decode_layer(queries=q.to(dev), key_states=nk.to(dev), value_states=nv.to(dev),
                                 entries=list(range(G)))
        ref = np.zeros((G, R, D))
        for e in range(G):
            pos = _quest_positions(model, e, q[e].float().numpy(), T + step, sink, recent, bs, budget_pages=8)
            for r in range(R):
                keys = torch.cat([model.keys[e][pos[r]], nk[e][None]]).float().numpy()
                vals = torch.cat([model.vals[e][pos[r]], nv[e][None]]).float().numpy()
                ref[e, r] = oracle.decode_attention(q[e, r:r + 1].float().numpy(), keys, vals, 1.0 / math.sqrt(D))[0]
            model.append(e, nk[e], nv[e])
        _close(out, ref)
    torch.cuda.synchronize()
    for e in range(G):
        assert _same(cache._key_cache[e, :T + 2], model.keys[e])


def test_quest_update_wide_group(H, dev):
    G, R, D, T, sink, recent, bs, frac = 2, 12, 64, 700, 16, 32, 16, 0.1
    _say("[wide quest update]")
    cache = H["quest"].QuestTopKOffloadedCache(num_cache_entries=G, max_cache_len=T + 4, head_dim=D,
                                               num_query_heads_per_kv=R, dtype=torch.bfloat16, device=dev,
                                               sink_tokens=sink, recent_tokens=recent, block_size=bs,
                                               budget_fraction=frac, kv_residency="host")
    model = _Model(G, T, D, "bf16", seed=103)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(104)
    for e in range(G):
        q = torch.randn(1, R, 1, D, generator=g).to(torch.bfloat16)
        nk, nv = model.new_token(D)
        K, V = cache.update(nk[None, None, None].to(dev), nv[None, None, None].to(dev), e,
                            {"query_states": q.to(dev)})
        lengths = cache.get_last_query_head_lengths(e)
        pos = _quest_positions(model, e, q[0, :, 0].float().numpy(), T, sink, recent, bs, frac=frac)
        assert lengths == tuple(len(p) + 1 for p in pos)
        for r in range(R):
            n = lengths[r]
            assert _same(K[0, r, :n - 1], model.keys[e][pos[r]]) and _same(K[0, r, n - 1], nk)


@pytest.mark.parametrize("R,mode", [(12, "matched"), (16, "dynamic")])
def test_twilight_gqa_group_union_wide_group(H, dev, R, mode):
    """Union of a 12- or 16-head group == unique(sink | every head's
    selection | recent) of the oracle, with matched budgets allocated over
    all R heads; then the GQA attention hook over it == float64."""
    G, D, T = 2, 128, 2000
    dtype = "bf16"
    _say(f"[wide twilight gqa] R={R} {mode}")
    cache = _twilight_cache(H, dev, E=G, T=T, D=D, R=R, dtype=dtype, residency="hbm", mode=mode,
                            candidate_token_budget=256, top_p=0.9, matched_budget_fraction=0.05,
                            layer_batched_selection=True, gqa_groupwise_execution=True, gpu_compact_gqa_union=True)
    model = _Model(G, T, D, dtype, seed=105, scale=2.0)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(106)
    entries = list(range(G))
    qs = [(torch.randn(1, R, 1, D, generator=g) * 2).to(torch.bfloat16) for _ in entries]
    new = [model.new_token(D) for _ in entries]
    cache.prepare_layer_selection(entries=entries, queries=[q.to(dev) for q in qs])
    K, V, cu, max_k, lengths = cache.update_layer_gqa_group_ragged(
        key_states=[k[None, None, None].to(dev) for k, _ in new],
        value_states=[v[None, None, None].to(dev) for _, v in new], queries=[q.to(dev) for q in qs], entries=entries)
    cu_h = cu.cpu().numpy()
    ref_out = np.zeros((G, R, D))
    for gi, e in enumerate(entries):
        ref = _twilight_expected(model, e, qs[gi][0, :, 0].float().numpy(), T, cache)
        s, n = int(cu_h[gi]), len(ref["union"])
        assert lengths[gi] == n + 1
        assert _same(K[s:s + n, 0], model.keys[e][ref["union"]])
        assert _same(K[s + n, 0], new[gi][0]) and _same(V[s + n, 0], new[gi][1])
        keys = torch.cat([model.keys[e][ref["union"]], new[gi][0][None]]).float().numpy()
        vals = torch.cat([model.vals[e][ref["union"]], new[gi][1][None]]).float().numpy()
        ref_out[gi] = oracle.decode_attention(qs[gi][0, :, 0].float().numpy(), keys, vals, 1.0 / math.sqrt(D))
    q_all = torch.cat([q[0, :, 0] for q in qs]).reshape(G, R, D).to(dev)
    out = H["mp"]._flash_attention_varlen_forward(q_all, K, V, torch.arange(G + 1, dtype=torch.int32, device=dev),
                                                  cu, 1, max_k, dropout=0.0, is_causal=True)
    _close(out, ref_out)


@pytest.mark.parametrize("mode", ["matched", "dynamic"])
def test_twilight_decode_layer_wide_group(H, dev, mode):
    """decode_layer with 16 query heads per KV head through the fused
    selection in two sub-groups of 8 whose records are ORed: dynamic budgets
    each head's own, matched budgets one allocation over all 16 heads (each
    sub-group's last launch reads every head's top-p count)."""
    G, R, D, T = 2, 16, 128, 1500
    _say(f"[wide twilight decode_layer] {mode}")
    cache = _twilight_cache(H, dev, E=G, T=T, D=D, R=R, dtype="f16", residency="hbm", mode=mode,
                            candidate_token_budget=256, top_p=0.9, matched_budget_fraction=0.05,
                            layer_batched_selection=True)
    model = _Model(G, T, D, "f16", seed=107, scale=2.0)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(108)
    q = (torch.randn(G, R, D, generator=g) * 2).to(torch.float16)
    new = [model.new_token(D) for _ in range(G)]
    nk = torch.stack([k for k, _ in new])
    nv = torch.stack([v for _, v in new])
    out = cache.decode_layer(queries=q.to(dev), key_states=nk.to(dev), value_states=nv.to(dev),
                             entries=list(range(G)))
    ref_out = np.zeros((G, R, D))
    for e in range(G):
        ref = _twilight_expected(model, e, q[e].float().numpy(), T, cache)
        keys = torch.cat([model.keys[e][ref["union"]], nk[e][None]]).float().numpy()
        vals = torch.cat([model.vals[e][ref["union"]], nv[e][None]]).float().numpy()
        ref_out[e] = oracle.decode_attention(q[e].float().numpy(), keys, vals, 1.0 / math.sqrt(D))
    _close(out, ref_out)
    torch.cuda.synchronize()
    assert _same(cache._key_cache[0, T], nk[0])
    assert cache._fused_bufs is not None   # the fused selection ran, not the general path

"""GPU tests of the offload caches' call surface against the CPU oracle.

Modelled on the reference's cache test (scripts/test_twilight_offload_cache_v1.py:
111-378): prefill through ``update``, then decode steps through each decode
entry point -- per-entry ``update`` (per-query-head packs), layer-batched
selection + ``update_layer_flat_ragged`` (per-head ragged segments),
``update_layer_gqa_group_ragged`` (one union per KV group) and the fused
``decode_layer`` fast path -- with the slab in pinned host memory or in HBM.
Gathered K/V must equal the oracle's selected rows bit for bit (plus the
decode token), union positions must equal the oracle's union, attention
outputs match a float64 reference within 2e-3 abs + 1e-2 rel, and every
appended token must land in the slab.
"""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

import oracle
from helpers import TORCH_DT, to_bits

pytestmark = pytest.mark.gpu


def _say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def H():
    import headinfer.mp as mp
    import headinfer.quest_offload_cache as qoc
    import headinfer.twilight_offload_cache as toc
    from headinfer import kernels

    return {"quest": qoc, "twilight": toc, "mp": mp, "kernels": kernels}


class _Model:
    """CPU copy of every entry's keys/values (prompt + appended tokens)."""

    def __init__(self, E, T, D, dtype, seed, scale=1.0):
        g = torch.Generator().manual_seed(seed)
        self.keys = [(torch.randn(T, D, generator=g) * scale).to(TORCH_DT[dtype]) for _ in range(E)]
        self.vals = [torch.randn(T, D, generator=g).to(TORCH_DT[dtype]) for _ in range(E)]
        self.prompt = T
        self.dtype = dtype
        self.gen = g

    def prefill(self, cache, dev):
        for e in range(len(self.keys)):
            k, v = cache.update(self.keys[e][None, None].to(dev), self.vals[e][None, None].to(dev), e)
            assert k.shape == (1, 1, self.prompt, self.keys[e].shape[1])

    def new_token(self, D):
        k = torch.randn(D, generator=self.gen).to(TORCH_DT[self.dtype])
        v = torch.randn(D, generator=self.gen).to(TORCH_DT[self.dtype])
        return k, v

    def append(self, e, k, v):
        self.keys[e] = torch.cat([self.keys[e], k[None]])
        self.vals[e] = torch.cat([self.vals[e], v[None]])


def _quest_positions(model, e, q, length, sink, recent, bs, frac=None, budget_pages=None):
    """Per-head positions of the Quest selection (oracle)."""
    kb = to_bits(model.keys[e][:model.prompt])
    pmin, pmax, _, _, _ = oracle.build_page_metadata(kb, model.dtype, sink, bs, quant=False)
    sink_end, recent_start, eligible = oracle.selection_window(length, sink, recent)
    cand = min(eligible // bs, pmin.shape[0])
    if budget_pages is not None:
        k = min(cand, budget_pages)
    else:
        k = min(cand, max(1, math.ceil(frac * eligible / bs)))
    R = q.shape[0]
    if k == 0:
        sel = np.zeros((R, 0), np.int64)
    else:
        sc = oracle.quest_score(q[None].astype(np.float32), pmin[None, :cand], pmax[None, :cand], model.dtype)[0]
        sel = oracle.topk_sorted(sc, k)
    return [np.concatenate([np.arange(sink_end), (sink + sel[r][:, None] * bs + np.arange(bs)).reshape(-1),
                            np.arange(recent_start, length)]).astype(np.int64) for r in range(R)]


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    a, b = a.detach().cpu().contiguous(), b.detach().cpu().contiguous()
    w = {2: torch.int16, 4: torch.int32}[a.element_size()]
    return a.shape == b.shape and torch.equal(a.view(w), b.view(w))


def _close(got, ref, atol=2e-3, rtol=1e-2):
    got = got.detach().float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    assert np.all(err <= atol + rtol * np.abs(ref)), f"max abs err {err.max():.3e}"


# ------------------------------------------------------------------ Quest
@pytest.mark.parametrize("residency,dtype", [("host", "f16"), ("hbm", "bf16")])
def test_quest_update_per_head_packs(H, dev, residency, dtype):
    """update(): each head's sink ++ pages ++ recent ++ decode token, bit-exact."""
    layers, G, R, D, T, sink, recent, bs, frac = 2, 2, 4, 128, 600, 16, 32, 16, 0.1
    E = layers * G
    _say(f"[quest update] {residency} {dtype}")
    cache = H["quest"].QuestTopKOffloadedCache(num_cache_entries=E, max_cache_len=T + 4, head_dim=D,
                                               num_query_heads_per_kv=R, dtype=TORCH_DT[dtype], device=dev,
                                               sink_tokens=sink, recent_tokens=recent, block_size=bs,
                                               budget_fraction=frac, kv_residency=residency)
    model = _Model(E, T, D, dtype, seed=7)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(8)
    for step in range(3):
        length = T + step
        for e in range(E):
            q = torch.randn(1, R, 1, D, generator=g).to(TORCH_DT[dtype])
            nk, nv = model.new_token(D)
            K, V = cache.update(nk[None, None, None].to(dev), nv[None, None, None].to(dev), e,
                                {"query_states": q.to(dev)})
            lengths = cache.get_last_query_head_lengths(e)
            pos = _quest_positions(model, e, q[0, :, 0].float().numpy(), length, sink, recent, bs, frac=frac)
            assert K.shape[:2] == (1, R) and lengths == tuple(len(p) + 1 for p in pos)
            for r in range(R):
                n = lengths[r]
                assert _same(K[0, r, :n - 1], model.keys[e][pos[r]]) and _same(V[0, r, :n - 1], model.vals[e][pos[r]])
                assert _same(K[0, r, n - 1], nk) and _same(V[0, r, n - 1], nv)
            model.append(e, nk, nv)
    torch.cuda.synchronize()
    for e in range(E):
        assert _same(cache._key_cache[e, :T + 3], model.keys[e]) and _same(cache._value_cache[e, :T + 3], model.vals[e])
    assert cache.get_seq_length(0) == T + 3 and cache.get_max_length() == T + 4


def test_quest_layer_flat_ragged_and_attention_hook(H, dev):
    """prepare_layer_selection + update_layer_flat_ragged == per-head segments;
    _flash_attention_varlen_forward over them == float64 attention."""
    layers, G, R, D, T, sink, recent, bs = 2, 4, 4, 128, 1500, 64, 256, 16
    E = layers * G
    dtype = "bf16"
    cache = H["quest"].QuestTopKOffloadedCache(num_cache_entries=E, max_cache_len=T + 2, head_dim=D,
                                               num_query_heads_per_kv=R, dtype=torch.bfloat16, device=dev,
                                               sink_tokens=sink, recent_tokens=recent, block_size=bs,
                                               budget_pages=20, layer_batched_selection=True,
                                               layer_flat_ragged_execution=True, kv_residency="hbm")
    model = _Model(E, T, D, dtype, seed=11)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(12)
    for layer in range(layers):
        entries = list(range(layer * G, layer * G + G))
        qs = [torch.randn(1, R, 1, D, generator=g).to(torch.bfloat16) for _ in entries]
        new = [model.new_token(D) for _ in entries]
        cache.prepare_layer_selection(entries=entries, queries=[q.to(dev) for q in qs])
        K, V, cu, max_k, lengths = cache.update_layer_flat_ragged(
            key_states=[k[None, None, None].to(dev) for k, _ in new],
            value_states=[v[None, None, None].to(dev) for _, v in new],
            queries=[q.to(dev) for q in qs], entries=entries)
        cu_h = cu.cpu().numpy()
        assert len(lengths) == G * R and cu_h[-1] == sum(lengths) and max_k == max(lengths)
        qflat = torch.cat([q[0, :, 0] for q in qs]).unsqueeze(1)  # [G*R, 1, D]
        out = H["mp"]._flash_attention_varlen_forward(qflat.to(dev), K, V,
                                                      torch.arange(G * R + 1, dtype=torch.int32, device=dev), cu,
                                                      1, max_k, dropout=0.0, is_causal=True)
        ref = np.zeros((G * R, 1, D))
        for gi, e in enumerate(entries):
            pos = _quest_positions(model, e, qs[gi][0, :, 0].float().numpy(), T, sink, recent, bs, budget_pages=20)
            for r in range(R):
                s = int(cu_h[gi * R + r])
                n = len(pos[r])
                assert lengths[gi * R + r] == n + 1
                assert _same(K[s:s + n, 0], model.keys[e][pos[r]]) and _same(V[s:s + n, 0], model.vals[e][pos[r]])
                assert _same(K[s + n, 0], new[gi][0]) and _same(V[s + n, 0], new[gi][1])
                keys = torch.cat([model.keys[e][pos[r]], new[gi][0][None]]).float().numpy()
                vals = torch.cat([model.vals[e][pos[r]], new[gi][1][None]]).float().numpy()
                ref[gi * R + r, 0] = oracle.decode_attention(qs[gi][0, r:r + 1, 0].float().numpy(), keys, vals,
                                                             1.0 / math.sqrt(D))[0]
            model.append(e, *new[gi])
        _close(out, ref)
    torch.cuda.synchronize()
    for e in range(E):
        assert _same(cache._key_cache[e, :T + 1], model.keys[e])


@pytest.mark.parametrize("residency", ["hbm", "host"])
def test_quest_decode_layer_fast_path(H, dev, residency):
    """decode_layer: union-plan attention straight from the slab with the
    fused append == per-head float64 attention over each head's rows."""
    G, R, D, T, sink, recent, bs = 8, 4, 128, 4096, 64, 256, 16
    dtype = "f16"
    _say(f"[quest decode_layer] {residency}")
    cache = H["quest"].QuestTopKOffloadedCache(num_cache_entries=G, max_cache_len=T + 2, head_dim=D,
                                               num_query_heads_per_kv=R, dtype=torch.float16, device=dev,
                                               sink_tokens=sink, recent_tokens=recent, block_size=bs,
                                               budget_pages=16, kv_residency=residency)
    model = _Model(G, T, D, dtype, seed=21)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(22)
    for step in range(2):
        q = torch.randn(G, R, D, generator=g).to(torch.float16)
        new = [model.new_token(D) for _ in range(G)]
        nk = torch.stack([k for k, _ in new])
        nv = torch.stack([v for _, v in new])
        out = cache.decode_layer(queries=q.to(dev), key_states=nk.to(dev), value_states=nv.to(dev),
                                 entries=list(range(G)))
        ref = np.zeros((G, R, D))
        for e in range(G):
            pos = _quest_positions(model, e, q[e].float().numpy(), T + step, sink, recent, bs, budget_pages=16)
            for r in range(R):
                keys = torch.cat([model.keys[e][pos[r]], nk[e][None]]).float().numpy()
                vals = torch.cat([model.vals[e][pos[r]], nv[e][None]]).float().numpy()
                ref[e, r] = oracle.decode_attention(q[e, r:r + 1].float().numpy(), keys, vals, 1.0 / math.sqrt(D))[0]
            model.append(e, nk[e], nv[e])
        _close(out, ref)
    torch.cuda.synchronize()
    for e in range(G):
        assert _same(cache._key_cache[e, :T + 2], model.keys[e]) and _same(cache._value_cache[e, :T + 2], model.vals[e])


@pytest.mark.parametrize("residency", ["hbm", "host"])
def test_quest_decode_metadata_update(H, dev, residency):
    """update_metadata_on_decode: pages completed during decode are scored
    and selected.  Decode keys are planted along the queries, so the pages
    they complete outrank the prompt's; the selection and the attention must
    match the oracle's over metadata of all rows, and the cache's metadata
    must equal a rebuild over the slab."""
    G, R, D, T, sink, recent, bs, steps = 2, 4, 128, 200, 16, 8, 16, 48
    dtype = "f16"
    _say(f"[quest metadata update] {residency}")
    cache = H["quest"].QuestTopKOffloadedCache(num_cache_entries=G, max_cache_len=T + steps, head_dim=D,
                                               num_query_heads_per_kv=R, dtype=torch.float16, device=dev,
                                               sink_tokens=sink, recent_tokens=recent, block_size=bs,
                                               budget_pages=4, kv_residency=residency,
                                               update_metadata_on_decode=True)
    model = _Model(G, T, D, dtype, seed=71)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(72)
    qdir = torch.randn(G, D, generator=g)
    qdir = qdir / qdir.norm(dim=1, keepdim=True)
    new_pages_selected = 0
    for step in range(steps):
        L = T + step
        q = (qdir[:, None, :] * 4 + 0.3 * torch.randn(G, R, D, generator=g)).to(torch.float16)
        nk = (qdir * 6 + 0.5 * torch.randn(G, D, generator=g)).to(torch.float16)
        nv = torch.randn(G, D, generator=g).to(torch.float16)
        out = cache.decode_layer(queries=q.to(dev), key_states=nk.to(dev), value_states=nv.to(dev),
                                 entries=list(range(G)))
        ref = np.zeros((G, R, D))
        for e in range(G):
            full = _Model.__new__(_Model)
            full.keys, full.prompt, full.dtype = model.keys, L, dtype
            pos = _quest_positions(full, e, q[e].float().numpy(), L, sink, recent, bs, budget_pages=4)
            new_pages_selected += sum(int((p >= T).sum()) for p in pos)
            for r in range(R):
                keys = torch.cat([model.keys[e][pos[r]], nk[e][None]]).float().numpy()
                vals = torch.cat([model.vals[e][pos[r]], nv[e][None]]).float().numpy()
                ref[e, r] = oracle.decode_attention(q[e, r:r + 1].float().numpy(), keys, vals, 1.0 / math.sqrt(D))[0]
            model.append(e, nk[e], nv[e])
        _close(out, ref)
    assert new_pages_selected > 0, "no page completed during decode was ever selected"
    torch.cuda.synchronize()
    pages = (T + steps - sink) // bs
    for e in range(G):
        omin, omax, _, _, _ = oracle.build_page_metadata(to_bits(model.keys[e]), dtype, sink, bs, quant=False)
        assert _same(cache._page_min[e, :pages], torch.from_numpy(omin.view(np.int16)).view(torch.float16))
        assert _same(cache._page_max[e, :pages], torch.from_numpy(omax.view(np.int16)).view(torch.float16))


# --------------------------------------------------------------- Twilight
def _twilight_expected(model, e, q, length, cache):
    kb = to_bits(model.keys[e][:model.prompt])
    pmin, pmax, packed, sc, mn = oracle.build_page_metadata(kb, model.dtype, cache.sink_tokens, cache.block_size)
    sink_end, recent_start, eligible = oracle.selection_window(length, cache.sink_tokens, cache.recent_tokens)
    bs = cache.block_size
    cand = min(eligible // bs, pmin.shape[0])
    fixed = min(cand, max(1, math.ceil(cache.matched_budget_fraction * eligible / bs)))
    b0 = min(cand, max(1, math.ceil(cache.candidate_token_budget / bs)))
    return oracle.twilight_layer(q.astype(np.float32), pmin[:cand], pmax[:cand], packed, sc, mn, model.dtype,
                                 length=length, sink=cache.sink_tokens, recent=cache.recent_tokens, block_size=bs,
                                 b0_pages=b0, top_p=cache.top_p, budget_mode=cache.budget_mode, fixed_pages=fixed)


def _twilight_cache(H, dev, *, E, T, D, R, dtype, residency, mode, **kw):
    return H["twilight"].TwilightMatchedBudgetOffloadedCache(
        num_cache_entries=E, max_cache_len=T + 4, head_dim=D, num_query_heads_per_kv=R, dtype=TORCH_DT[dtype],
        device=dev, kv_residency=residency, budget_mode=mode, **kw)


@pytest.mark.parametrize("residency,dtype,mode", [("host", "bf16", "matched"), ("hbm", "f16", "dynamic")])
def test_twilight_gqa_group_union(H, dev, residency, dtype, mode):
    """update_layer_gqa_group_ragged: K/V == slab[union] ++ decode token,
    union == unique(sink | per-head selections | recent) of the oracle."""
    layers, G, R, D, T = 2, 4, 4, 128, 3000
    E = layers * G
    _say(f"[twilight gqa] {residency} {dtype} {mode}")
    cache = _twilight_cache(H, dev, E=E, T=T, D=D, R=R, dtype=dtype, residency=residency, mode=mode,
                            candidate_token_budget=512, top_p=0.9, matched_budget_fraction=0.05,
                            layer_batched_selection=True, gqa_groupwise_execution=True, gpu_compact_gqa_union=True)
    model = _Model(E, T, D, dtype, seed=31, scale=2.0)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(32)
    for step in range(2):
        for layer in range(layers):
            entries = list(range(layer * G, layer * G + G))
            qs = [(torch.randn(1, R, 1, D, generator=g) * 2).to(TORCH_DT[dtype]) for _ in entries]
            new = [model.new_token(D) for _ in entries]
            cache.prepare_layer_selection(entries=entries, queries=[q.to(dev) for q in qs])
            K, V, cu, max_k, lengths = cache.update_layer_gqa_group_ragged(
                key_states=[k[None, None, None].to(dev) for k, _ in new],
                value_states=[v[None, None, None].to(dev) for _, v in new],
                queries=[q.to(dev) for q in qs], entries=entries)
            cu_h = cu.cpu().numpy()
            assert cu_h[0] == 0 and list(np.diff(cu_h)) == list(lengths) and max_k == max(lengths)
            for gi, e in enumerate(entries):
                ref = _twilight_expected(model, e, qs[gi][0, :, 0].float().numpy(), T + step, cache)
                s, n = int(cu_h[gi]), len(ref["union"])
                assert lengths[gi] == n + 1, (gi, lengths[gi], n)
                assert _same(K[s:s + n, 0], model.keys[e][ref["union"]])
                assert _same(V[s:s + n, 0], model.vals[e][ref["union"]])
                assert _same(K[s + n, 0], new[gi][0]) and _same(V[s + n, 0], new[gi][1])
                model.append(e, *new[gi])
    torch.cuda.synchronize()
    for e in range(E):
        assert _same(cache._key_cache[e, :T + 2], model.keys[e])


@pytest.mark.parametrize("mode", ["matched", "dynamic"])
def test_twilight_gqa_group_union_resident_cache(H, dev, mode):
    """update_layer_gqa_group_ragged with previous_token_resident_cache (the
    reference's path for it): K/V == slab[oracle union] ++ decode token at
    every step, although before each step the cache's host slab copies of the
    previous step's union rows are overwritten with noise -- a row packed
    again must come from the HBM copy of the previous step; rows are counted
    as hits, some are, and the slab gets every append."""
    layers, G, R, D, T, steps = 2, 4, 4, 128, 3000, 4
    E = layers * G
    dtype = "bf16"
    _say(f"[twilight gqa resident] {mode}")
    cache = _twilight_cache(H, dev, E=E, T=T, D=D, R=R, dtype=dtype, residency="host", mode=mode,
                            candidate_token_budget=512, top_p=0.9, matched_budget_fraction=0.05,
                            layer_batched_selection=True, gqa_groupwise_execution=True, cpu_flat_gather=True,
                            direct_attention_layout=True, gather_h2d_chunks=1, previous_token_resident_cache=True)
    model = _Model(E, T, D, dtype, seed=33, scale=2.0)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(34)
    noise = torch.Generator().manual_seed(35)
    bases = [torch.randn(1, R, 1, D, generator=g) * 2 for _ in range(E)]
    prev_union = [None] * E
    for step in range(steps):
        torch.cuda.synchronize()
        for e in range(E):   # the slab back to the model's rows, then the previous union to noise
            n = T + step
            cache._key_cache[e, :n] = model.keys[e][:n]
            cache._value_cache[e, :n] = model.vals[e][:n]
            if prev_union[e] is not None:
                m = len(prev_union[e])
                cache._key_cache[e, prev_union[e]] = torch.randn((m, D), generator=noise).to(torch.bfloat16)
                cache._value_cache[e, prev_union[e]] = torch.randn((m, D), generator=noise).to(torch.bfloat16)
        for layer in range(layers):
            entries = list(range(layer * G, layer * G + G))
            qs = [(bases[e] + 0.3 * torch.randn(1, R, 1, D, generator=g)).to(TORCH_DT[dtype]) for e in entries]
            new = [model.new_token(D) for _ in entries]
            cache.prepare_layer_selection(entries=entries, queries=[q.to(dev) for q in qs])
            K, V, cu, max_k, lengths = cache.update_layer_gqa_group_ragged(
                key_states=[k[None, None, None].to(dev) for k, _ in new],
                value_states=[v[None, None, None].to(dev) for _, v in new],
                queries=[q.to(dev) for q in qs], entries=entries)
            cu_h = cu.cpu().numpy()
            assert cu_h[0] == 0 and list(np.diff(cu_h)) == list(lengths) and max_k == max(lengths)
            for gi, e in enumerate(entries):
                ref = _twilight_expected(model, e, qs[gi][0, :, 0].float().numpy(), T + step, cache)
                s, n = int(cu_h[gi]), len(ref["union"])
                assert lengths[gi] == n + 1, (gi, lengths[gi], n)
                assert _same(K[s:s + n, 0], model.keys[e][ref["union"]]), (step, e)
                assert _same(V[s:s + n, 0], model.vals[e][ref["union"]]), (step, e)
                assert _same(K[s + n, 0], new[gi][0]) and _same(V[s + n, 0], new[gi][1])
                model.append(e, *new[gi])
                prev_union[e] = torch.as_tensor(np.asarray(ref["union"]), dtype=torch.long)
            torch.cuda.synchronize()
            for gi, e in enumerate(entries):   # the append landed in the slab
                assert _same(cache._key_cache[e, T + step], new[gi][0]), (step, e)
                assert _same(cache._value_cache[e, T + step], new[gi][1]), (step, e)
    st = cache.resident_stats()
    _say(f"[twilight gqa resident] {st}")
    assert 0 < st["resident_hit_pages"] < st["union_pages"], st


def test_twilight_decode_metadata_update(H, dev):
    """Twilight with update_metadata_on_decode: decode rows get INT4 codes and
    completed pages get min/max, so the union over pages completed during
    decode equals the oracle's over metadata of all rows."""
    G, R, D, T, steps = 2, 4, 128, 300, 40
    dtype = "bf16"
    _say("[twilight metadata update]")
    cache = H["twilight"].TwilightMatchedBudgetOffloadedCache(
        num_cache_entries=G, max_cache_len=T + steps, head_dim=D, num_query_heads_per_kv=R,
        dtype=torch.bfloat16, device=dev, kv_residency="hbm", budget_mode="dynamic", sink_tokens=16,
        recent_tokens=8, block_size=16, candidate_token_budget=64, top_p=0.9, layer_batched_selection=True,
        gqa_groupwise_execution=True, gpu_compact_gqa_union=True, update_metadata_on_decode=True)
    model = _Model(G, T, D, dtype, seed=81)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(82)
    qdir = torch.randn(G, D, generator=g)
    qdir = qdir / qdir.norm(dim=1, keepdim=True)
    entries = list(range(G))
    late = 0
    for step in range(steps):
        L = T + step
        qs = [(qdir[e] * 4 + 0.3 * torch.randn(R, D, generator=g)).to(torch.bfloat16)[None, :, None] for e in entries]
        new = [((qdir[e] * 6 + 0.5 * torch.randn(D, generator=g)).to(torch.bfloat16),
                torch.randn(D, generator=g).to(torch.bfloat16)) for e in entries]
        cache.prepare_layer_selection(entries=entries, queries=[q.to(dev) for q in qs])
        K, V, cu, max_k, lengths = cache.update_layer_gqa_group_ragged(
            key_states=[k[None, None, None].to(dev) for k, _ in new],
            value_states=[v[None, None, None].to(dev) for _, v in new],
            queries=[q.to(dev) for q in qs], entries=entries)
        cu_h = cu.cpu().numpy()
        for gi, e in enumerate(entries):
            full = _Model.__new__(_Model)
            full.keys, full.prompt, full.dtype = model.keys, L, dtype
            ref = _twilight_expected(full, e, qs[gi][0, :, 0].float().numpy(), L, cache)
            u = np.asarray(ref["union"])
            prompt_pages_end = 16 + ((T - 16) // 16) * 16  # rows of pages complete at prefill
            late += int(((u >= prompt_pages_end) & (u < L - 7)).sum())  # pages completed during decode
            s0, n = int(cu_h[gi]), len(ref["union"])
            assert lengths[gi] == n + 1, (step, gi, lengths[gi], n)
            assert _same(K[s0:s0 + n, 0], model.keys[e][ref["union"]])
            model.append(e, *new[gi])
    assert late > 0


@pytest.mark.parametrize("residency,dtype,fused,mode", [("hbm", "f16", True, "dynamic"), ("host", "bf16", True, "dynamic"),
                                                        ("hbm", "bf16", False, "dynamic"),
                                                        ("hbm", "bf16", True, "matched"),
                                                        ("host", "f16", True, "matched"),
                                                        ("hbm", "f16", False, "matched")])
def test_twilight_decode_layer(H, dev, residency, dtype, fused, mode):
    """decode_layer: every head of a group attends the oracle's group union ++
    the decode token (float64 reference), with dynamic or matched budgets,
    through the fused selection (union record) or the union-row path, and the
    decode tokens land in the slab."""
    G, R, D, T, steps = 4, 4, 128, 3000, 3
    _say(f"[twilight decode_layer] {residency} {dtype} fused={fused} {mode}")
    cache = _twilight_cache(H, dev, E=G, T=T, D=D, R=R, dtype=dtype, residency=residency, mode=mode,
                            candidate_token_budget=512, top_p=0.9, matched_budget_fraction=0.05)
    cache.fused_decode = fused
    model = _Model(G, T, D, dtype, seed=51, scale=2.0)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(52)
    for step in range(steps):
        q = (torch.randn(G, R, D, generator=g) * 2).to(TORCH_DT[dtype])
        new = [model.new_token(D) for _ in range(G)]
        nk = torch.stack([k for k, _ in new])
        nv = torch.stack([v for _, v in new])
        out = cache.decode_layer(queries=q.to(dev), key_states=nk.to(dev), value_states=nv.to(dev),
                                 entries=list(range(G)))
        ref = np.zeros((G, R, D))
        for e in range(G):
            union = np.asarray(_twilight_expected(model, e, q[e].float().numpy(), T + step, cache)["union"])
            keys = torch.cat([model.keys[e][union], nk[e][None]]).float().numpy()
            vals = torch.cat([model.vals[e][union], nv[e][None]]).float().numpy()
            for r in range(R):
                ref[e, r] = oracle.decode_attention(q[e, r:r + 1].float().numpy(), keys, vals, 1.0 / math.sqrt(D))[0]
            model.append(e, nk[e], nv[e])
        _close(out, ref)
    torch.cuda.synchronize()
    for e in range(G):
        n = T + steps
        assert _same(cache._key_cache[e, :n], model.keys[e]) and _same(cache._value_cache[e, :n], model.vals[e])


@pytest.mark.parametrize("mode", ["dynamic", "matched"])
def test_twilight_decode_layer_resident_cache(H, dev, mode):
    """previous_token_resident_cache on a Twilight cache with a host slab
    (with the execution flags the reference requires for it): decode_layer
    == the same cache without it, bit for bit, over 4 steps of drifting
    queries, while kept rows of the previous step come from the HBM resident
    cache (counted: some rows hit) and the slabs receive the same appends."""
    G, R, D, T, steps = 4, 4, 128, 3000, 4
    _say(f"[twilight resident decode_layer] {mode}")
    kw = dict(candidate_token_budget=512, top_p=0.9, matched_budget_fraction=0.05)
    flags = dict(previous_token_resident_cache=True, layer_batched_selection=True, gqa_groupwise_execution=True,
                 cpu_flat_gather=True, direct_attention_layout=True, gather_h2d_chunks=1)
    res_cache = _twilight_cache(H, dev, E=G, T=T, D=D, R=R, dtype="bf16", residency="host", mode=mode, **kw, **flags)
    plain = _twilight_cache(H, dev, E=G, T=T, D=D, R=R, dtype="bf16", residency="host", mode=mode, **kw)
    assert res_cache._resident_active and not plain._resident_active
    model = _Model(G, T, D, "bf16", seed=61, scale=2.0)
    model.prefill(res_cache, dev)
    model.prefill(plain, dev)
    g = torch.Generator().manual_seed(62)
    base = torch.randn(G, R, D, generator=g) * 2
    for step in range(steps):
        q = (base + 0.3 * torch.randn(G, R, D, generator=g)).to(torch.bfloat16).to(dev)
        new = [model.new_token(D) for _ in range(G)]
        nk = torch.stack([k for k, _ in new]).to(dev)
        nv = torch.stack([v for _, v in new]).to(dev)
        a = res_cache.decode_layer(queries=q, key_states=nk, value_states=nv, entries=list(range(G)))
        b = plain.decode_layer(queries=q, key_states=nk, value_states=nv, entries=list(range(G)))
        torch.cuda.synchronize()
        assert _same(a, b), step
    n = T + steps
    assert _same(res_cache._key_cache[:, :n], plain._key_cache[:, :n])
    assert _same(res_cache._value_cache[:, :n], plain._value_cache[:, :n])
    st = res_cache.resident_stats()
    _say(f"[twilight resident decode_layer] {st}")
    assert 0 < st["resident_hit_pages"] < st["union_pages"], st


def test_twilight_per_head_update_and_flat(H, dev):
    """Per-entry update() and update_layer_flat_ragged give every head its own
    Twilight selection (the oracle's per-head selected positions)."""
    G, R, D, T = 2, 3, 64, 1200
    dtype = "bf16"
    cache = _twilight_cache(H, dev, E=G, T=T, D=D, R=R, dtype=dtype, residency="host", mode="matched",
                            sink_tokens=16, recent_tokens=32, block_size=8, candidate_token_budget=400, top_p=0.8,
                            matched_budget_fraction=0.1)
    model = _Model(G, T, D, dtype, seed=41, scale=2.0)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(42)
    for e in range(G):
        q = (torch.randn(1, R, 1, D, generator=g) * 2).to(torch.bfloat16)
        nk, nv = model.new_token(D)
        K, V = cache.update(nk[None, None, None].to(dev), nv[None, None, None].to(dev), e, {"query_states": q.to(dev)})
        ref = _twilight_expected(model, e, q[0, :, 0].float().numpy(), T, cache)
        sink_end, recent_start, _ = oracle.selection_window(T, cache.sink_tokens, cache.recent_tokens)
        lengths = cache.get_last_query_head_lengths(e)
        for r in range(R):
            pos = np.concatenate([np.arange(sink_end), ref["selected"][r], np.arange(recent_start, T)])
            assert lengths[r] == len(pos) + 1
            assert _same(K[0, r, :len(pos)], model.keys[e][pos]) and _same(K[0, r, len(pos)], nk)
            assert _same(V[0, r, :len(pos)], model.vals[e][pos])
        model.append(e, nk, nv)

    flat = _twilight_cache(H, dev, E=G, T=T, D=D, R=R, dtype=dtype, residency="hbm", mode="dynamic",
                           sink_tokens=16, recent_tokens=32, block_size=8, candidate_token_budget=400, top_p=0.8,
                           layer_batched_selection=True, layer_flat_ragged_execution=True)
    model = _Model(G, T, D, dtype, seed=43, scale=2.0)
    model.prefill(flat, dev)
    qs = [(torch.randn(1, R, 1, D, generator=g) * 2).to(torch.bfloat16) for _ in range(G)]
    new = [model.new_token(D) for _ in range(G)]
    flat.prepare_layer_selection(entries=list(range(G)), queries=[q.to(dev) for q in qs])
    K, V, cu, max_k, lengths = flat.update_layer_flat_ragged(
        key_states=[k[None, None, None].to(dev) for k, _ in new], value_states=[v[None, None, None].to(dev) for _, v in new],
        queries=[q.to(dev) for q in qs], entries=list(range(G)))
    cu_h = cu.cpu().numpy()
    sink_end, recent_start, _ = oracle.selection_window(T, 16, 32)
    for e in range(G):
        ref = _twilight_expected(model, e, qs[e][0, :, 0].float().numpy(), T, flat)
        for r in range(R):
            pos = np.concatenate([np.arange(sink_end), ref["selected"][r], np.arange(recent_start, T)])
            s = int(cu_h[e * R + r])
            assert lengths[e * R + r] == len(pos) + 1
            assert _same(K[s:s + len(pos), 0], model.keys[e][pos]) and _same(K[s + len(pos), 0], new[e][0])


def test_twilight_tiny_fixture(H, dev):
    """The reference test's tiny fixture shape (2 entries, max_cache_len 32,
    D=4, R=3, bf16, sink 1, recent 2, block 1, B0=8, seed 1234) through the
    GQA group path."""
    E, T, D, R = 2, 28, 4, 3
    cache = _twilight_cache(H, dev, E=E, T=T, D=D, R=R, dtype="bf16", residency="host", mode="matched",
                            sink_tokens=1, recent_tokens=2, block_size=1, candidate_token_budget=8, top_p=0.9,
                            matched_budget_fraction=0.25, layer_batched_selection=True, gqa_groupwise_execution=True)
    model = _Model(E, T, D, "bf16", seed=1234)
    model.prefill(cache, dev)
    g = torch.Generator().manual_seed(1234)
    qs = [torch.randn(1, R, 1, D, generator=g).to(torch.bfloat16) for _ in range(E)]
    new = [model.new_token(D) for _ in range(E)]
    cache.prepare_layer_selection(entries=[0, 1], queries=[q.to(dev) for q in qs])
    K, V, cu, max_k, lengths = cache.update_layer_gqa_group_ragged(
        key_states=[k[None, None, None].to(dev) for k, _ in new], value_states=[v[None, None, None].to(dev) for _, v in new],
        queries=[q.to(dev) for q in qs], entries=[0, 1])
    cu_h = cu.cpu().numpy()
    for e in range(E):
        ref = _twilight_expected(model, e, qs[e][0, :, 0].float().numpy(), T, cache)
        s, n = int(cu_h[e]), len(ref["union"])
        assert lengths[e] == n + 1 and _same(K[s:s + n, 0], model.keys[e][ref["union"]])


# ------------------------------------------------------------- operators
@pytest.mark.parametrize("dtype,D", [("bf16", 128), ("f16", 4), ("f32", 256)])
def test_fused_affine_int4_qk(H, dev, dtype, D):
    """fused_affine_int4_qk at explicit positions == the oracle's INT4 QK
    (qk_scale 1, bit-exact); materialize == the oracle's dequantized rows."""
    K = H["kernels"]
    G, R, T, N = 3, 4, 500, 77
    gen = torch.Generator().manual_seed(D)
    keys = (torch.randn(G, T, D, generator=gen) * 2).to(TORCH_DT[dtype])
    packed = torch.empty((G, T, D // 2), dtype=torch.uint8, device=dev)
    sc = torch.empty((G, T), dtype=TORCH_DT[dtype], device=dev)
    mn = torch.empty_like(sc)
    K.build_page_metadata(keys.to(dev), sink=T, block_size=1, packed=packed, scale=sc, minimum=mn)
    q = torch.randn(G, R, D, generator=gen)
    pos = torch.randint(0, T, (G, R, N), generator=gen)
    got = K.fused_affine_int4_qk(q.to(dev), packed, sc, mn, pos.to(dev))
    mat = K.fused_affine_int4_qk(q.to(dev), packed, sc, mn, pos.to(dev), materialize=True)
    torch.cuda.synchronize()
    kb = to_bits(keys)
    for g in range(G):
        _, _, pk, s_, m_ = oracle.build_page_metadata(kb[g], dtype, T, 1, pages=False)
        deq = oracle.int4_dequantize(pk, s_, m_, dtype)
        for r in range(R):
            want = oracle.int4_qk(q[g, r].numpy(), pk, s_, m_, dtype, pos[g, r].numpy(), 1.0)
            assert np.array_equal(got[g, r].cpu().numpy().view(np.uint32), want.view(np.uint32))
            assert np.array_equal(mat[g, r].cpu().numpy().view(np.uint32), deq[pos[g, r].numpy()].view(np.uint32))


def test_quest_previous_token_resident_cache(H, dev):
    """previous_token_resident_cache on a host slab: decode_layer outputs and
    slab contents equal the plain cache's, and later steps hit the HBM
    resident pages."""
    G, R, D, T, steps = 4, 4, 128, 3000, 6
    dtype = "f16"
    _say("[quest resident cache]")
    kw = dict(num_cache_entries=G, max_cache_len=T + steps + 2, head_dim=D, num_query_heads_per_kv=R,
              dtype=torch.float16, device=dev, budget_pages=16, kv_residency="host")
    plain = H["quest"].QuestTopKOffloadedCache(**kw)
    res = H["quest"].QuestTopKOffloadedCache(previous_token_resident_cache=True, **kw)
    model = _Model(G, T, D, dtype, seed=121)
    model.prefill(plain, dev)
    model.prefill(res, dev)
    g = torch.Generator().manual_seed(122)
    base = torch.randn(G, R, D, generator=g)
    for step in range(steps):
        q = (base + 0.1 * torch.randn(G, R, D, generator=g)).to(torch.float16).to(dev)
        new = [model.new_token(D) for _ in range(G)]
        nk = torch.stack([k for k, _ in new]).to(dev)
        nv = torch.stack([v for _, v in new]).to(dev)
        a = res.decode_layer(queries=q, key_states=nk, value_states=nv, entries=list(range(G)))
        b = plain.decode_layer(queries=q, key_states=nk, value_states=nv, entries=list(range(G)))
        torch.cuda.synchronize()
        assert _same(a, b), step
    n = T + steps  # the rows past it were never written (stale pinned memory)
    assert _same(res._key_cache[:, :n], plain._key_cache[:, :n])
    assert _same(res._value_cache[:, :n], plain._value_cache[:, :n])
    st = res.resident_stats()
    assert 0 < st["resident_hit_pages"] < st["union_pages"], st

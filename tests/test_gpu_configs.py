"""Two measured configurations at their full sizes, checked against the oracle.

* 64K host offload: a Llama-3-8B-shaped cache of 32 layers x 8 KV heads
  (head_dim 128, bf16) with the whole slab in pinned host memory, 65 536-token
  prompts and a Quest budget of 128 pages (2048 tokens) per query head.  The
  slab is 2 x 256 entries x 65 544 rows x 256 B = 8.6 GB: the V plane starts
  2^32 + 0.5 MB bytes in, and the last entry's top 2048 rows (its recent
  window, decode rows and late pages) lie past 2^32 bytes of the K plane.  Layers 0 and 31 carry seeded
  random keys; their selection (the cache's own page metadata, scored and
  ranked by the kernel) must equal the oracle's bit for bit, their decode_layer
  attention (zero-copy reads over the host link, the append fused) must match
  float64 over the oracle's rows, and the ragged page-tile kernels the graph
  decoder runs must do the same on the last layer.
* Multi-request decode: 8 requests of 16K-131K tokens (seed 4) on a
  Qwen2.5-7B-like GQA shape (28 query / 4 KV heads, head_dim 128, bf16),
  KV heads {0, 1} in HBM and {2, 3} in pinned host memory, the step (ragged
  select, ragged page-tile attention with the append, ragged metadata update,
  device-side length increment) replayed from one captured graph.  After the
  eager step and after graph replays, every group's union plan must equal the
  union of the oracle's per-head top-k at the group's own length, its
  attention must match float64 over its rows, and the page metadata must equal
  a rebuild over the slab.
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from helpers import to_bits

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def _say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def _union_plan(sel_heads: np.ndarray):
    union = np.unique(sel_heads.reshape(-1))
    masks = np.zeros(union.shape[0], np.uint8)
    for r in range(sel_heads.shape[0]):
        masks[np.searchsorted(union, sel_heads[r])] |= np.uint8(1 << r)
    return union, masks


def _attention64(q: np.ndarray, keys: np.ndarray, vals: np.ndarray) -> np.ndarray:
    return oracle.decode_attention(q, keys, vals, 1.0 / math.sqrt(q.shape[-1]))


def _close(got, ref, what):
    got = np.asarray(got, dtype=np.float64)
    err = np.abs(got - ref)
    assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), f"{what}: max abs err {err.max():.3e}"


# ----------------------------------------------------------- 64K host offload
def test_offload64k_host_slab_past_4gib(dev):
    from headinfer import kernels
    from headinfer.quest_offload_cache import QuestTopKOffloadedCache

    layers, G, R, D, T = 32, 8, 4, 128, 65536
    sink, recent, bs, k = 64, 256, 16, 128
    steps = 2
    E = layers * G
    _say("[offload64k] building the 8.6 GB pinned slab")
    cache = QuestTopKOffloadedCache(num_cache_entries=E, max_cache_len=T + 8, head_dim=D, num_query_heads_per_kv=R,
                                    dtype=torch.bfloat16, device=dev, sink_tokens=sink, recent_tokens=recent,
                                    block_size=bs, budget_pages=k, kv_residency="host")
    row_bytes = D * 2
    # the K plane crosses 2^32 bytes at row 63 496 of the last entry, below
    # its recent window and decode rows; the V plane starts past it
    assert cache.geometry.row(E - 1, 0) * row_bytes < 2 ** 32 <= cache.geometry.row(E - 1, T - 2000) * row_bytes
    assert cache._value_cache.data_ptr() - cache._key_cache.data_ptr() >= 2 ** 32
    tested = (0, layers - 1)
    gen = torch.Generator(device=dev).manual_seed(40)
    filler = torch.randn((2, T, D), generator=gen, device=dev).to(torch.bfloat16)
    keys = {}
    for layer in range(layers):
        for g in range(G):
            e = layer * G + g
            if layer in tested:
                kv = torch.randn((2, T, D), generator=gen, device=dev).to(torch.bfloat16)
                keys[e] = kv[0].cpu()
            else:
                kv = filler
            cache.update(kv[0][None, None], kv[1][None, None], e)
    torch.cuda.synchronize()
    _say("[offload64k] prefill done")
    hg = torch.Generator().manual_seed(41)
    for step in range(steps):
        L = T + step
        sink_end, recent_start, eligible = oracle.selection_window(L, sink, recent)
        cand = min(eligible // bs, cache._page_min.shape[1])
        kk = min(cand, k)
        for layer in range(layers):
            e0 = layer * G
            q = torch.randn((G, R, D), generator=hg).to(torch.bfloat16)
            nk = torch.randn((G, D), generator=hg).to(torch.bfloat16)
            nv = torch.randn((G, D), generator=hg).to(torch.bfloat16)
            if layer in tested:
                sel = torch.empty((G, R, kk), dtype=torch.int32, device=dev)
                kernels.quest_select(q.float().to(dev), cache._page_min[e0:e0 + G, :cand],
                                     cache._page_max[e0:e0 + G, :cand], kk, sel_pages=sel)
            out = cache.decode_layer(queries=q.to(dev), key_states=nk.to(dev), value_states=nv.to(dev),
                                     entries=list(range(e0, e0 + G)))
            if layer not in tested:
                continue
            torch.cuda.synchronize()
            sel_h = sel.cpu().numpy()
            ref = np.zeros((G, R, D))
            for g in range(G):
                e = e0 + g
                kb = to_bits(keys[e])
                omin, omax, _, _, _ = oracle.build_page_metadata(kb, "bf16", sink, bs, quant=False)
                sc = oracle.quest_score(q[g][None].float().numpy(), omin[None, :cand], omax[None, :cand], "bf16")[0]
                want = oracle.topk_sorted(sc, kk)
                assert np.array_equal(sel_h[g], want), (layer, g)
                slab_rows = cache._key_cache[e]          # pinned host [Lmax, D]
                assert torch.equal(slab_rows[L].view(torch.int16), nk[g].view(torch.int16))
                assert torch.equal(cache._value_cache[e, L].view(torch.int16), nv[g].view(torch.int16))
                for r in range(R):
                    rows = np.concatenate([np.arange(sink_end), (sink + want[r][:, None] * bs + np.arange(bs)).ravel(),
                                           np.arange(recent_start, L + 1)])
                    kr = cache._key_cache[e][torch.from_numpy(rows)].float().numpy()
                    vr = cache._value_cache[e][torch.from_numpy(rows)].float().numpy()
                    ref[g, r] = _attention64(q[g, r:r + 1].float().numpy(), kr, vr)[0]
                keys[e] = torch.cat([keys[e], nk[g][None]])
            _close(out.float().cpu().numpy(), ref, f"decode_layer layer {layer} step {step}")
            if layer == layers - 1:
                # the graph decoder's ragged kernels on the same rows past 4 GiB
                lengths = torch.full((G,), L, dtype=torch.int32, device=dev)
                width = min(cand, R * kk)
                pp = torch.empty((G, width), dtype=torch.int32, device=dev)
                pm = torch.empty((G, width), dtype=torch.uint8, device=dev)
                pc = torch.empty((G,), dtype=torch.int32, device=dev)
                kernels.quest_select_ragged(q.float().to(dev), cache._page_min[e0:e0 + G],
                                            cache._page_max[e0:e0 + G], lengths, kk, sink=sink, recent=recent,
                                            block_size=bs, plan_pages=pp, plan_masks=pm, plan_counts=pc)
                rag = kernels.decode_attention_pages_ragged(
                    q.to(dev), cache._key_cache[e0:e0 + G], cache._value_cache[e0:e0 + G], pp, pc, lengths,
                    plan_masks=pm, max_pages=width, sink=sink, recent=recent, block_size=bs, append=False,
                    cur_k=nk.to(dev), cur_v=nv.to(dev))
                torch.cuda.synchronize()
                for g in range(G):
                    want = oracle.topk_sorted(oracle.quest_score(
                        q[g][None].float().numpy(), *[m[None, :cand] for m in oracle.build_page_metadata(
                            to_bits(keys[e0 + g][:L]), "bf16", sink, bs, quant=False)[:2]], "bf16")[0], kk)
                    union, masks = _union_plan(want)
                    n = int(pc[g])
                    assert n == union.shape[0] and np.array_equal(pp[g, :n].cpu().numpy(), union)
                    assert np.array_equal(pm[g, :n].cpu().numpy(), masks)
                _close(rag.float().cpu().numpy(), ref, f"ragged page-tile attention layer {layer} step {step}")
        _say(f"[offload64k] step {step} ok")
    del cache


# ------------------------------------------------------ multi-request decode
def _bench():
    if str(ROOT) not in sys.path:
        sys.path.insert(0, str(ROOT))
    import bench

    return bench


def _check_plans(w, layer: int):
    """Every group's union plan of `layer` (both residency sets) == the union
    of the oracle's per-head top-k over the pages complete before its length."""
    lens = [L - 1 for L in w.lengths.tolist()]
    for s in ("hbm", "host"):
        pp, pm, pc = (t.cpu().numpy() for t in w.plan[layer][s])
        e0 = layer * w.G
        q = w.qf[layer][s].cpu().numpy()
        for gi, L in enumerate(lens):
            keys = w.slab[s][0, e0 + gi, :L].cpu()
            omin, omax, _, _, _ = oracle.build_page_metadata(to_bits(keys), "bf16", w.SINK, w.BS, quant=False)
            _, _, eligible = oracle.selection_window(L, w.SINK, w.RECENT)
            P = min(eligible // w.BS, w.P)
            kk = min(w.BUDGET, P)
            sc = oracle.quest_score(q[gi][None], omin[None, :P], omax[None, :P], "bf16")[0]
            union, masks = _union_plan(oracle.topk_sorted(sc, kk))
            n = int(pc[gi])
            assert n == union.shape[0], (s, gi, L)
            assert np.array_equal(pp[gi, :n], union) and np.array_equal(pm[gi, :n], masks), (s, gi, L)


def test_multireq_full_contexts_graph_replays(dev):
    bench = _bench()
    _say("[multireq] building 8 requests x 2 layers")
    w = bench.MultiRequestWorkload(dev, layers=2)
    assert max(w.contexts) > 117000 and w.R == 7
    w.step()
    torch.cuda.synchronize()
    _check_plans(w, 0)
    ok, err = bench.multireq_check(w)
    assert ok, f"eager step: attention/metadata mismatch (max abs err {err:.3e})"
    _say("[multireq] eager step ok")
    g = bench.graph_of(w.step, warm=0)
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        if rep in (0, 3):
            _check_plans(w, 0)
            _check_plans(w, 1)
            ok, err = bench.multireq_check(w)
            assert ok, f"replay {rep}: attention/metadata mismatch (max abs err {err:.3e})"
            _say(f"[multireq] replay {rep} ok")
    assert w.lengths.tolist() == [L + 5 for L in w.lengths0]

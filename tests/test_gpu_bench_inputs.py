"""The measured workloads' own inputs against the oracle.

bench.py times the sparse-decode step on structured inputs: the 32K Quest
layer has 16 planted pages aligned with the query and 4 outlier channels x8
(the 4K one the same at k = 16); the 32K Twilight layer adds Zipf(1.1) page
relevance to its keys.  Those peaked distributions are what stresses the
one-pass histogram fast paths of the top-k and top-p, so the selections the
timed step makes are held to the oracle here, on the same seeded inputs,
for two layers at full size:

* Quest: every head's selected pages (the selection bitmaps the attention
  ranks) == oracle.topk_sorted(oracle.quest_score(...)) bit for bit
  (quest_offload_cache.py:362-374), and each head's attention output
  within 2e-3 abs + 1e-2 rel of float64 over sink ++ its pages ++ recent ++
  the decode token (mp.py:239-279);
* Twilight, dynamic and matched budgets: the union record's kept rows ==
  oracle.twilight_layer's union, the top-p counts equal, and the union
  attention within the same tolerance of float64 over the oracle's rows
  (twilight_offload_cache.py:1144-1354)."""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

import oracle
from helpers import to_bits

pytestmark = pytest.mark.gpu


def _say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def _close(got: np.ndarray, ref: np.ndarray, what: str) -> None:
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), f"{what}: max abs err {err.max():.3e}"


@pytest.mark.parametrize("context,budget", [(4096, 16), (32768, 128)])
def test_quest_workload_selection_and_attention_match_oracle(dev, context, budget):
    import bench

    layers = 2
    _say(f"[bench inputs] quest context={context} k={budget}: building")
    w = bench.QuestWorkload(dev, layers, context, budget)
    w.step()
    torch.cuda.synchronize()
    G, R, D, P, L = w.G, w.R, w.D, w.P, w.L
    sink_end, recent_start, _ = oracle.selection_window(L, w.SINK, w.RECENT)
    for layer in range(layers):
        q = w.qf[layer].cpu().numpy()
        sc = oracle.quest_score(q, to_bits(w.pmin[layer, :, :P]), to_bits(w.pmax[layer, :, :P]), "f16")
        ref_sel = oracle.topk_sorted(sc.reshape(G * R, P), w.k).reshape(G, R, w.k)
        words = w.bits[layer].cpu().numpy().view(np.uint32)
        p = np.arange(P)
        got = ((words[:, :, p >> 5] >> (p & 31).astype(np.uint32)) & 1).astype(bool)   # [G, R, P]
        out = w.out[layer].float().cpu().numpy()
        kc, vc = w.kc[layer].float(), w.vc[layer].float()
        for g in range(G):
            for r in range(R):
                assert np.array_equal(np.flatnonzero(got[g, r]), ref_sel[g, r]), (layer, g, r)
                pages = torch.from_numpy(ref_sel[g, r]).long()
                rows = torch.cat([torch.arange(sink_end),
                                  (w.SINK + pages[:, None] * w.BS + torch.arange(w.BS)).reshape(-1),
                                  torch.arange(recent_start, L)]).to(kc.device)
                keys = torch.cat([kc[g, rows], w.cur_k[layer, g:g + 1].float()]).cpu().numpy()
                vals = torch.cat([vc[g, rows], w.cur_v[layer, g:g + 1].float()]).cpu().numpy()
                ref = oracle.decode_attention(q[g, r:r + 1], keys, vals, 1.0 / math.sqrt(D))
                _close(out[g, r:r + 1], ref, f"quest attention layer {layer} group {g} head {r}")
        _say(f"[bench inputs] quest layer {layer} ok")


@pytest.mark.parametrize("mode", ["dynamic", "matched"])
def test_twilight_workload_selection_and_attention_match_oracle(dev, mode):
    import bench

    layers = 2
    _say(f"[bench inputs] twilight 32K {mode}: building")
    w = bench.TwilightWorkload(dev, layers, 32768, mode)
    w.step()
    torch.cuda.synchronize()
    G, R, D, P, L = w.G, w.R, w.D, w.P, w.L
    for layer in range(layers):
        out = w.out[layer].float().cpu().numpy()
        des = w.desired[layer].cpu().numpy()
        for g in range(G):
            ref = oracle.twilight_layer(w.qf[layer, g].cpu().numpy(), to_bits(w.pmin[layer, g, :P]),
                                        to_bits(w.pmax[layer, g, :P]), w.packed[layer, g].cpu().numpy(),
                                        to_bits(w.scale[layer, g]), to_bits(w.minimum[layer, g]), "bf16", length=L,
                                        sink=w.SINK, recent=w.RECENT, block_size=w.BS, b0_pages=w.b0,
                                        top_p=w.TOP_P, budget_mode=mode, fixed_pages=w.fixed)
            assert np.array_equal(des[g], ref["desired"]), (layer, g, des[g], ref["desired"])
            kept = w.kept_rows(layer, g).cpu().numpy()
            assert np.array_equal(kept, ref["union"]), (layer, g, kept.size, ref["union"].size)
            if mode == "matched":
                assert int(ref["allocated"].sum()) == w.fixed * w.BS * R
            rows = torch.from_numpy(ref["union"].astype(np.int64)).to(w.kc.device)
            keys = torch.cat([w.kc[layer, g, rows].float(), w.cur_k[layer, g:g + 1].float()]).cpu().numpy()
            vals = torch.cat([w.vc[layer, g, rows].float(), w.cur_v[layer, g:g + 1].float()]).cpu().numpy()
            ref_o = oracle.decode_attention(w.qf[layer, g].cpu().numpy(), keys, vals, 1.0 / math.sqrt(D))
            _close(out[g], ref_o, f"twilight {mode} attention layer {layer} group {g}")
        _say(f"[bench inputs] twilight {mode} layer {layer} ok: desired {des[0].tolist()}")

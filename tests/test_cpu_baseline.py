"""The CPU baseline port (oracle/cpu_baseline.py) times the right
computation: on a tie-free input its Quest pages are the oracle's top-k of the
oracle's scores, and its attention output matches float64 attention over each
head's selected rows plus the decode token.  CPU only."""

from __future__ import annotations

import math

import numpy as np
import torch

import oracle
from helpers import to_bits
from oracle.cpu_baseline import quest_layer_step


def test_quest_layer_step_selects_the_oracle_pages():
    G, R, D, L, sink, recent, bs, k = 2, 4, 64, 900, 16, 32, 16, 6
    gen = torch.Generator().manual_seed(11)
    keys = torch.randn((G, L, D), generator=gen).to(torch.float16)
    vals = torch.randn((G, L, D), generator=gen).to(torch.float16)
    q = torch.randn((G, R, D), generator=gen).to(torch.float16)
    cur_k = torch.randn((G, D), generator=gen).to(torch.float16)
    cur_v = torch.randn((G, D), generator=gen).to(torch.float16)
    sink_end, recent_start, eligible = oracle.selection_window(L, sink, recent)
    P = eligible // bs
    pmin = torch.empty((G, P, D), dtype=torch.float16)
    pmax = torch.empty_like(pmin)
    for g in range(G):
        mn, mx, _, _, _ = oracle.build_page_metadata(to_bits(keys[g]), "f16", sink, bs, quant=False)
        pmin[g] = torch.from_numpy(mn[:P].view(np.int16)).view(torch.float16)
        pmax[g] = torch.from_numpy(mx[:P].view(np.int16)).view(torch.float16)
    phases: dict = {}
    out, chosen = quest_layer_step(q, keys, vals, pmin, pmax, cur_k, cur_v, length=L, budget=k, sink=sink,
                                   recent=recent, block_size=bs, phases=phases)
    assert set(phases) == {"score_select", "gather", "attention"} and all(v >= 0 for v in phases.values())
    for g in range(G):
        sc = oracle.quest_score(q[g].float().numpy()[None], to_bits(pmin[g])[None], to_bits(pmax[g])[None], "f16")[0]
        srt = np.sort(sc, axis=1)
        assert (np.diff(srt, axis=1) != 0).all(), "the input must be tie-free"
        want = oracle.topk_sorted(sc, k)
        assert np.array_equal(chosen[g].numpy(), want)
        for r in range(R):
            rows = np.concatenate([np.arange(sink_end), (sink + want[r][:, None] * bs + np.arange(bs)).ravel(),
                                   np.arange(recent_start, L)])
            kk = torch.cat([keys[g, rows], cur_k[g:g + 1]]).float().numpy()
            vv = torch.cat([vals[g, rows], cur_v[g:g + 1]]).float().numpy()
            ref = oracle.decode_attention(q[g, r:r + 1].float().numpy(), kk, vv, 1.0 / math.sqrt(D))[0]
            assert np.abs(out[g, r].float().numpy() - ref).max() <= 2e-3 + 1e-2 * np.abs(ref).max()

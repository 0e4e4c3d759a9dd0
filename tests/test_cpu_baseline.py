"""The CPU baseline port (oracle/cpu_baseline.py) times the right
computation: on a tie-free input its Quest pages are the oracle's top-k of the
oracle's scores, and its attention output matches float64 attention over each
head's selected rows plus the decode token.  CPU only."""

from __future__ import annotations

import math

import numpy as np
import pytest
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


@pytest.mark.parametrize("mode,fixed", [("dynamic", 0), ("matched", 5)])
def test_twilight_layer_step_follows_the_oracle(mode, fixed):
    """The Twilight port takes the oracle's B0 pages, and its per-group union
    differs from oracle.twilight_layer's only by the rows its fp32
    dequantize/matmul/softmax/cumsum puts on the other side of a count (the
    reference's order, unpinned; the oracle's is the exact-integer rule):
    at most a few rows per head.  With matched budgets the kept rows per head
    are the largest-remainder allocation of fixed pages x 16 x R."""
    from oracle.cpu_baseline import twilight_layer_step

    G, R, D, L, sink, recent, bs, b0 = 2, 4, 128, 2000, 64, 256, 16, 24
    gen = torch.Generator().manual_seed(5)
    keys = (torch.randn((G, L, D), generator=gen) * 1.5).to(torch.bfloat16)
    vals = torch.randn((G, L, D), generator=gen).to(torch.bfloat16)
    q = (torch.randn((G, R, D), generator=gen) * 2).to(torch.bfloat16)
    cur_k = torch.randn((G, D), generator=gen).to(torch.bfloat16)
    cur_v = torch.randn((G, D), generator=gen).to(torch.bfloat16)
    P = oracle.selection_window(L, sink, recent)[2] // bs
    meta = [oracle.build_page_metadata(to_bits(keys[g]), "bf16", sink, bs) for g in range(G)]

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)

    pmin = torch.stack([t(m[0][:P]) for m in meta])
    pmax = torch.stack([t(m[1][:P]) for m in meta])
    packed = torch.stack([torch.from_numpy(m[2]) for m in meta])
    scale = torch.stack([t(m[3]) for m in meta])
    minimum = torch.stack([t(m[4]) for m in meta])
    phases: dict = {}
    out, unions = twilight_layer_step(q, keys, vals, pmin, pmax, packed, scale, minimum, cur_k, cur_v, length=L,
                                      b0_pages=b0, top_p=0.9, sink=sink, recent=recent, block_size=bs,
                                      budget_mode=mode, fixed_pages=fixed, phases=phases)
    assert set(phases) == {"score_select", "int4_qk", "top_p", "union", "gather", "attention"}
    for g in range(G):
        ref = oracle.twilight_layer(q[g].float().numpy(), meta[g][0][:P], meta[g][1][:P], meta[g][2], meta[g][3],
                                    meta[g][4], "bf16", length=L, sink=sink, recent=recent, block_size=bs,
                                    b0_pages=b0, top_p=0.9, budget_mode=mode, fixed_pages=fixed)
        got = set(unions[g].tolist())
        want = set(ref["union"].tolist())
        assert len(got ^ want) <= 3 * R, (g, len(got ^ want))
        kept = unions[g].numpy()
        kk = torch.cat([keys[g, kept], cur_k[g:g + 1]]).float().numpy()
        vv = torch.cat([vals[g, kept], cur_v[g:g + 1]]).float().numpy()
        ref_o = oracle.decode_attention(q[g].float().numpy(), kk, vv, 1.0 / math.sqrt(D))
        assert np.abs(out[g].float().numpy() - ref_o).max() <= 2e-3 + 1e-2 * np.abs(ref_o).max()

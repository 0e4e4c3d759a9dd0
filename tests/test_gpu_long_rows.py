"""Selection over rows longer than one block holds (P > 8192 pages: contexts
past 131K tokens at 16-token pages).  The top-k goes through a segment pass
(each 8192-page segment keeps its own top k) and a selection over the
compacted row, and the union plan through a page bitmap.  Everything is
checked against the oracle bit for bit: page ids (ties to the lowest page
across segment edges, NaN highest), the union plan and the row plan, ragged
groups whose lengths straddle segment edges, and the error for a compacted
row that would not fit a block."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import oracle
from helpers import minmax_pages, randn, to_bits

pytestmark = pytest.mark.gpu


def _say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def K():
    from headinfer import kernels

    return kernels


def _score_rows(P: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    rows = [torch.randn(P, generator=g),
            torch.randint(-3, 4, (P,), generator=g).float(),       # ties across every segment edge
            torch.full((P,), 1.5)]                                  # one value: lowest pages win
    r = torch.randn(P, generator=g)
    r[P - 1] = float("nan")                                         # NaN ranks highest, in the last segment
    r[8191:8194] = -0.0
    rows.append(r)
    return torch.stack(rows)


@pytest.mark.parametrize("P", [8193, 20000, 65536])
def test_topk_sorted_long_rows(K, dev, P):
    _say(f"[long topk] P={P}")
    s = _score_rows(P, P)
    for k in (1, 128, 1000):
        want = oracle.topk_sorted(s.numpy(), k)
        got = K.topk_sorted(s.to(dev), k)
        assert np.array_equal(got.cpu().numpy(), want), k
        wide = torch.zeros((s.shape[0], P + 3))                     # strided rows: the scalar load path
        wide[:, :P] = s
        got2 = K.topk_sorted(wide.to(dev)[:, :P], k)
        assert np.array_equal(got2.cpu().numpy(), want), ("strided", k)


def test_long_row_width_limit(K, dev):
    # 2 full segments and 1 page: 2 * 4096 + 1 compacted keys > 8192
    s = torch.randn((1, 16385))
    with pytest.raises(RuntimeError):
        K.topk_sorted(s.to(dev), 4096)
    got = K.topk_sorted(s.to(dev), 4000)                            # 8001 keys: fits
    assert np.array_equal(got.cpu().numpy(), oracle.topk_sorted(s.numpy(), 4000))


def _quantized_pages(G: int, P: int, D: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    lo = torch.randint(-2, 3, (G, P, D), generator=g).to(torch.bfloat16)
    hi = lo + torch.randint(0, 2, (G, P, D), generator=g).to(torch.bfloat16)
    return lo, hi


@pytest.mark.parametrize("P,k,G,R,dtype,ties", [
    (16384, 128, 2, 4, "bf16", False),
    (16384, 256, 2, 4, "bf16", True),
    (65536, 128, 1, 4, "bf16", False),
    (20000, 64, 1, 8, "f16", False),
])
def test_quest_select_long_rows(K, dev, P, k, G, R, dtype, ties):
    sink, recent, bs, D = 64, 256, 16, 128
    L = sink + P * bs + recent - 1                                  # exactly P whole pages are eligible
    _say(f"[long quest_select] P={P} k={k} G={G} R={R} {dtype} ties={ties} L={L}")
    lo, hi = _quantized_pages(G, P, D, P + k) if ties else minmax_pages(dtype, G, P, D, seed=P + k)
    q = randn((G, R, D), "f32", seed=P + 1)
    if ties:
        q = q.sign()                                                 # integer-valued scores: many equal pages
    sel = torch.empty((G, R, k), dtype=torch.int32, device=dev)
    pw = min(P, R * k)
    ppages = torch.full((G, pw), -3, dtype=torch.int32, device=dev)
    pmasks = torch.zeros((G, pw), dtype=torch.uint8, device=dev)
    pcounts = torch.zeros((G,), dtype=torch.int32, device=dev)
    rows = torch.full((G, L + 1), -7, dtype=torch.int32, device=dev)
    rmasks = torch.zeros((G, L + 1), dtype=torch.uint8, device=dev)
    rcounts = torch.zeros((G,), dtype=torch.int32, device=dev)
    for _ in range(2):                                               # the arrival counters reset themselves
        K.quest_select(q.to(dev), lo.to(dev), hi.to(dev), k, sel_pages=sel, plan_pages=ppages, plan_masks=pmasks,
                       plan_counts=pcounts, rows=rows, row_masks=rmasks, row_counts=rcounts, sink=sink,
                       recent=recent, block_size=bs, length=L, append_position=L)
        torch.cuda.synchronize()
    ref_scores = oracle.quest_score(q.numpy(), to_bits(lo), to_bits(hi), dtype)
    ref_sel = oracle.topk_sorted(ref_scores, k)
    assert np.array_equal(sel.cpu().numpy(), ref_sel)
    for g in range(G):
        union = np.unique(ref_sel[g])
        nu = int(pcounts[g])
        assert nu == len(union) and np.array_equal(ppages[g, :nu].cpu().numpy(), union)
        want = np.zeros(len(union), np.uint8)
        for r in range(R):
            want[np.searchsorted(union, ref_sel[g, r])] |= np.uint8(1 << r)
        assert np.array_equal(pmasks[g, :nu].cpu().numpy(), want)
        r_rows, r_masks = oracle.quest_row_plan(ref_sel[g], P, sink, recent, bs, L, L)
        n = int(rcounts[g])
        assert n == len(r_rows)
        assert np.array_equal(rows[g, :n].cpu().numpy(), r_rows)
        assert np.array_equal(rmasks[g, :n].cpu().numpy(), r_masks)


def test_quest_select_ragged_long_rows(K, dev):
    """Groups whose page counts sit below k, at and just past a segment edge,
    inside a later segment and at P_max."""
    sink, recent, bs, D, R, k = 64, 256, 16, 128, 4, 128
    P_max = 20000
    pages = [50, 8192, 8193, 12345, 16389, P_max]
    G = len(pages)
    lengths = [sink + p * bs + recent - 1 + (g % bs) for g, p in enumerate(pages)]
    _say(f"[long ragged] pages {pages}")
    lo, hi = minmax_pages("bf16", G, P_max, D, seed=77)
    q = randn((G, R, D), "f32", seed=78)
    sel = torch.full((G, R, k), -5, dtype=torch.int32, device=dev)
    pw = min(P_max, R * k)
    ppages = torch.full((G, pw), -3, dtype=torch.int32, device=dev)
    pmasks = torch.zeros((G, pw), dtype=torch.uint8, device=dev)
    pcounts = torch.zeros((G,), dtype=torch.int32, device=dev)
    lens = torch.tensor(lengths, dtype=torch.int32, device=dev)
    for _ in range(2):
        K.quest_select_ragged(q.to(dev), lo.to(dev), hi.to(dev), lens, k, sink=sink, recent=recent, block_size=bs,
                              sel_pages=sel, plan_pages=ppages, plan_masks=pmasks, plan_counts=pcounts)
        torch.cuda.synchronize()
    lo_b, hi_b = to_bits(lo), to_bits(hi)
    for g, L in enumerate(lengths):
        _, _, eligible = oracle.selection_window(L, sink, recent)
        P = min(eligible // bs, P_max)
        assert P == pages[g]
        kk = min(k, P)
        sc = oracle.quest_score(q[g][None].numpy(), lo_b[g][None, :P], hi_b[g][None, :P], "bf16")[0]
        want = oracle.topk_sorted(sc, kk)
        got = sel[g].cpu().numpy()
        assert np.array_equal(got[:, :kk], want), g
        assert np.all(got[:, kk:] == -1), g
        union = np.unique(want)
        nu = int(pcounts[g])
        assert nu == len(union) and np.array_equal(ppages[g, :nu].cpu().numpy(), union), g
        m = np.zeros(len(union), np.uint8)
        for r in range(R):
            m[np.searchsorted(union, want[r])] |= np.uint8(1 << r)
        assert np.array_equal(pmasks[g, :nu].cpu().numpy(), m), g

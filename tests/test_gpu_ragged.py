"""GPU parity of the ragged (multi-request) entry points.

Groups of one launch have different lengths, read from a device array:
quest_select_ragged and the ragged Twilight stage 2 must equal the oracle at
each group's own length (bit-exact page ids, union plan, logits, counts and
union rows), the ragged page-tile
attention must match float64 attention over each group's own window, and the
ragged metadata update must equal a rebuild.  A decode step made of these
launches plus the device-side length increment is captured in a HIP graph
and every replay is checked against the same step run eagerly.
"""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

import oracle
from helpers import from_bits, randn, same_bits, to_bits

pytestmark = pytest.mark.gpu

SINK, RECENT, BS, D = 64, 256, 16, 128


def _say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def K():
    from headinfer import kernels

    return kernels


def _metadata(keys, lengths, dtype, dev):
    """Page min/max [G, P_max, D] of each group's complete pages over its own rows."""
    G, Lmax, _ = keys.shape
    P_max = (Lmax - SINK) // BS
    pmin = torch.zeros((G, P_max, D), dtype=keys.dtype)
    pmax = torch.zeros_like(pmin)
    for g in range(G):
        kb = to_bits(keys[g, :lengths[g]])
        omin, omax, _, _, _ = oracle.build_page_metadata(kb, dtype, SINK, BS, quant=False)
        if omin.shape[0]:
            pmin[g, :omin.shape[0]] = from_bits(omin, dtype)
            pmax[g, :omax.shape[0]] = from_bits(omax, dtype)
    return pmin.to(dev), pmax.to(dev)


def _cand(L):
    sink_end, recent_start, eligible = oracle.selection_window(L, SINK, RECENT)
    return eligible // BS


LENGTHS = [40, 400, 1000, 5000, 20000, 33000]


def _oracle_plan(sel_heads: np.ndarray):
    """Union plan of a group from its heads' page lists: ascending union
    pages and the bitmask of the heads that chose each."""
    union = np.unique(sel_heads.reshape(-1))
    masks = np.zeros(union.shape[0], np.uint8)
    for r in range(sel_heads.shape[0]):
        masks[np.searchsorted(union, sel_heads[r])] |= np.uint8(1 << r)
    return union, masks


@pytest.mark.parametrize("dtype,R", [("bf16", 7), ("f16", 4)])
def test_quest_select_ragged_matches_oracle(K, dev, dtype, R):
    """Each group of the ragged launch == the oracle's Quest score + top-k at
    that group's own length (bit-exact page ids), and its union plan == the
    set union of its heads' pages with the heads' bitmask."""
    _say(f"[ragged select] {dtype} R={R}")
    G, k = len(LENGTHS), 128
    Lmax = max(LENGTHS) + 16
    keys = randn((G, Lmax, D), dtype, seed=91)
    q = randn((G, R, D), "f32", seed=92)
    pmin, pmax = _metadata(keys, LENGTHS, dtype, dev)
    P_max = pmin.shape[1]
    lengths = torch.tensor(LENGTHS, dtype=torch.int32, device=dev)
    width = min(P_max, R * k)
    sel = torch.empty((G, R, k), dtype=torch.int32, device=dev)
    pp = torch.empty((G, width), dtype=torch.int32, device=dev)
    pm = torch.empty((G, width), dtype=torch.uint8, device=dev)
    pc = torch.empty((G,), dtype=torch.int32, device=dev)
    K.quest_select_ragged(q.to(dev), pmin, pmax, lengths, k, sink=SINK, recent=RECENT, block_size=BS, sel_pages=sel,
                          plan_pages=pp, plan_masks=pm, plan_counts=pc)
    torch.cuda.synchronize()
    pmin_h, pmax_h = to_bits(pmin), to_bits(pmax)
    for g, L in enumerate(LENGTHS):
        P = _cand(L)
        kg = min(k, P)
        assert bool((sel[g, :, kg:] == -1).all()), g
        if P == 0:
            assert int(pc[g]) == 0
            continue
        sc = oracle.quest_score(q[g:g + 1].numpy(), pmin_h[g:g + 1, :P], pmax_h[g:g + 1, :P], dtype)[0]
        want = oracle.topk_sorted(sc, kg)
        assert np.array_equal(sel[g, :, :kg].cpu().numpy(), want), g
        union, masks = _oracle_plan(want)
        n = int(pc[g])
        assert n == union.shape[0], g
        assert np.array_equal(pp[g, :n].cpu().numpy(), union) and np.array_equal(pm[g, :n].cpu().numpy(), masks), g


def _rows(L, pages, masks, R, decode):
    sink_end, recent_start, _ = oracle.selection_window(L, SINK, RECENT)
    pg = pages.long()
    rows = torch.cat([torch.arange(sink_end), (SINK + pg[:, None] * BS + torch.arange(BS)).reshape(-1),
                      torch.arange(recent_start, L)])
    all_heads = (1 << R) - 1
    m = np.concatenate([np.full(sink_end, all_heads), masks.long().repeat_interleave(BS).numpy(),
                        np.full(L - recent_start, all_heads)])
    if decode != "none":
        m = np.concatenate([m, [all_heads]])
    return rows, m.astype(np.uint8)


@pytest.mark.parametrize("decode", ["cur_append", "cache_row", "none"])
@pytest.mark.parametrize("dtype,R", [("bf16", 7), ("f16", 4)])
def test_decode_attention_pages_ragged(K, dev, dtype, R, decode):
    _say(f"[ragged attention] {dtype} R={R} decode={decode}")
    G, k = len(LENGTHS), 128
    Lmax = max(LENGTHS) + 16
    keys = randn((G, Lmax, D), dtype, seed=93)
    vals = randn((G, Lmax, D), dtype, seed=94)
    q = randn((G, R, D), dtype, seed=95)
    ck, cv = randn((G, D), dtype, seed=96), randn((G, D), dtype, seed=97)
    pmin, pmax = _metadata(keys, LENGTHS, dtype, dev)
    lengths = torch.tensor(LENGTHS, dtype=torch.int32, device=dev)
    width = min(pmin.shape[1], R * k)
    pp = torch.empty((G, width), dtype=torch.int32, device=dev)
    pm = torch.empty((G, width), dtype=torch.uint8, device=dev)
    pc = torch.empty((G,), dtype=torch.int32, device=dev)
    K.quest_select_ragged(q.float().to(dev), pmin, pmax, lengths, k, sink=SINK, recent=RECENT, block_size=BS,
                          plan_pages=pp, plan_masks=pm, plan_counts=pc)
    kd, vd = keys.to(dev), vals.to(dev)
    kw = dict(plan_masks=pm, max_pages=width, sink=SINK, recent=RECENT, block_size=BS)
    if decode == "cur_append":
        kw.update(append=True, cur_k=ck.to(dev), cur_v=cv.to(dev))
    else:
        kw.update(append=decode == "cache_row")
    out = K.decode_attention_pages_ragged(q.to(dev), kd, vd, pp, pc, lengths, **kw)
    torch.cuda.synchronize()
    ref = np.zeros((G, R, D))
    for g, L in enumerate(LENGTHS):
        n = int(pc[g])
        rows, m = _rows(L, pp[g, :n].cpu(), pm[g, :n].cpu(), R, decode)
        kk, vv = keys[g, rows], vals[g, rows]
        if decode == "cur_append":
            kk, vv = torch.cat([kk, ck[g:g + 1]]), torch.cat([vv, cv[g:g + 1]])
            assert same_bits(kd[g, L], ck[g]) and same_bits(vd[g, L], cv[g]), g
        elif decode == "cache_row":
            kk, vv = torch.cat([kk, keys[g, L:L + 1]]), torch.cat([vv, vals[g, L:L + 1]])
        ref[g] = oracle.decode_attention(q[g].float().numpy(), kk.float().numpy(), vv.float().numpy(),
                                         1.0 / math.sqrt(D), m)
    if decode != "cur_append":
        assert same_bits(kd, keys.to(dev)) and same_bits(vd, vals.to(dev))
    got = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), f"max abs err {err.max():.3e}"


def test_update_page_metadata_ragged(K, dev):
    _say("[ragged metadata update]")
    dtype = "bf16"
    E, Lmax = 4, 400
    keys = randn((E, Lmax, D), dtype, seed=98)
    starts = [100, 143, 200, 300]
    kd = keys.to(dev)
    P = (Lmax - SINK) // BS
    pmin = torch.zeros((E, P, D), dtype=keys.dtype, device=dev)
    pmax = torch.zeros_like(pmin)
    packed = torch.zeros((E, Lmax, D // 2), dtype=torch.uint8, device=dev)
    scale = torch.zeros((E, Lmax), dtype=keys.dtype, device=dev)
    minimum = torch.zeros_like(scale)
    for e, T in enumerate(starts):
        K.build_page_metadata(kd[e, :T], sink=SINK, block_size=BS, page_min=pmin[e], page_max=pmax[e],
                              packed=packed[e], scale=scale[e], minimum=minimum[e])
    pos = torch.tensor(starts, dtype=torch.int32, device=dev)
    steps = 40
    for _ in range(steps):
        K.update_page_metadata_ragged(kd, pos, first_entry=0, sink=SINK, block_size=BS, page_min=pmin,
                                      page_max=pmax, packed=packed, scale=scale, minimum=minimum)
        pos += 1
    # a row beyond the buffers is skipped, not written
    K.update_page_metadata_ragged(kd, torch.tensor([-1, Lmax, Lmax + 5, -7], dtype=torch.int32, device=dev),
                                  first_entry=0, sink=SINK, block_size=BS, page_min=pmin, page_max=pmax,
                                  packed=packed, scale=scale, minimum=minimum)
    torch.cuda.synchronize()
    for e, T in enumerate(starts):
        n = T + steps
        omin, omax, opk, osc, omn = oracle.build_page_metadata(to_bits(keys[e, :n]), dtype, SINK, BS)
        p = omin.shape[0]
        assert same_bits(pmin[e, :p], from_bits(omin, dtype)) and same_bits(pmax[e, :p], from_bits(omax, dtype)), e
        assert bool((pmin[e, p:] == 0).all()), e
        assert np.array_equal(packed[e, :n].cpu().numpy(), opk), e
        assert same_bits(scale[e, :n], from_bits(osc, dtype)) and same_bits(minimum[e, :n], from_bits(omn, dtype))
        assert bool((packed[e, n:] == 0).all()), e


def test_ragged_step_graph_replays_match_eager(K, dev):
    """select + attention (append) + metadata update + length increment,
    captured once and replayed; each replay == the eager step, bit for bit."""
    _say("[ragged graph]")
    dtype, R, k = "bf16", 7, 32
    lengths0 = [700, 1500, 2222, 3001]
    G = len(lengths0)
    steps = 5
    Lmax = max(lengths0) + steps + 16
    keys = randn((G, Lmax, D), dtype, seed=101)
    vals = randn((G, Lmax, D), dtype, seed=102)
    q = randn((G, R, D), dtype, seed=103)
    ck, cv = randn((G, D), dtype, seed=104), randn((G, D), dtype, seed=105)
    P_cap = (Lmax - SINK) // BS

    def state():
        pmin, pmax = _metadata(keys, lengths0, dtype, dev)
        st = {"k": keys.to(dev), "v": vals.to(dev), "pmin": pmin, "pmax": pmax,
              "len": torch.tensor(lengths0, dtype=torch.int32, device=dev),
              "pp": torch.zeros((G, min(P_cap, R * k)), dtype=torch.int32, device=dev),
              "pm": torch.zeros((G, min(P_cap, R * k)), dtype=torch.uint8, device=dev),
              "pc": torch.zeros((G,), dtype=torch.int32, device=dev),
              "out": torch.zeros((G, R, D), dtype=q.dtype, device=dev),
              "q": q.to(dev), "qf": q.float().to(dev), "ck": ck.to(dev), "cv": cv.to(dev)}
        return st

    def step(st):
        K.quest_select_ragged(st["qf"], st["pmin"], st["pmax"], st["len"], k, sink=SINK, recent=RECENT,
                              block_size=BS, plan_pages=st["pp"], plan_masks=st["pm"], plan_counts=st["pc"])
        K.decode_attention_pages_ragged(st["q"], st["k"], st["v"], st["pp"], st["pc"], st["len"],
                                        plan_masks=st["pm"], max_pages=st["pp"].shape[1], sink=SINK, recent=RECENT,
                                        block_size=BS, append=True, cur_k=st["ck"], cur_v=st["cv"], out=st["out"])
        K.update_page_metadata_ragged(st["k"], st["len"], first_entry=0, sink=SINK, block_size=BS,
                                      page_min=st["pmin"], page_max=st["pmax"])
        st["len"].add_(1)

    eager, graphed = state(), state()
    step(graphed)  # warm-up (workspaces) outside the capture, then restore the graphed state
    torch.cuda.synchronize()
    ref_state = state()
    for name in ("k", "v", "pmin", "pmax", "len"):
        graphed[name].copy_(ref_state[name])
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            step(graphed)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    # capture recorded but did not run the step: the graphed state is still at step 0
    assert torch.equal(graphed["len"].cpu(), eager["len"].cpu())
    for i in range(steps):
        step(eager)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(graphed["len"].cpu(), eager["len"].cpu()), i
        assert torch.equal(graphed["pc"].cpu(), eager["pc"].cpu()), i
        assert same_bits(graphed["out"], eager["out"]), i
        assert same_bits(graphed["k"], eager["k"]) and same_bits(graphed["pmin"], eager["pmin"]), i


@pytest.mark.parametrize("ragged", [True, False])
def test_resident_page_cache_bit_exact(K, dev, ragged):
    """Host slab, several decode steps with drifting queries: attention with
    the HBM resident page cache == without it, bit for bit; the resident
    buffer holds the slab's pages at their union indices; hits are counted."""
    _say(f"[resident pages] ragged={ragged}")
    dtype, R, k, steps = "bf16", 4, 16, 5
    lengths0 = [3000, 3000, 3000] if not ragged else [2500, 3100, 4000]
    G = len(lengths0)
    Lmax = max(lengths0) + steps + 16
    keys = randn((G, Lmax, D), dtype, seed=111)
    vals = randn((G, Lmax, D), dtype, seed=112)
    kh, vh = keys.clone().pin_memory(), vals.clone().pin_memory()      # resident-cache run (host slab)
    kh2, vh2 = keys.clone().pin_memory(), vals.clone().pin_memory()    # plain run (host slab)
    pmin, pmax = _metadata(keys, lengths0, dtype, dev)
    P = pmin.shape[1]
    width = min(P, R * k)
    res = K.ResidentPages(G, width, P, D, keys.dtype, dev)
    lengths = torch.tensor(lengths0, dtype=torch.int32, device=dev)
    g = torch.Generator().manual_seed(113)
    base = torch.randn((G, R, D), generator=g)
    for step in range(steps):
        q = (base + 0.15 * torch.randn((G, R, D), generator=g)).to(torch.bfloat16)
        ck, cv = randn((G, D), dtype, seed=200 + step), randn((G, D), dtype, seed=300 + step)
        pp = torch.zeros((G, width), dtype=torch.int32, device=dev)
        pm = torch.zeros((G, width), dtype=torch.uint8, device=dev)
        pc = torch.zeros((G,), dtype=torch.int32, device=dev)
        K.quest_select_ragged(q.float().to(dev), pmin, pmax, lengths, k, sink=SINK, recent=RECENT, block_size=BS,
                              plan_pages=pp, plan_masks=pm, plan_counts=pc)
        kw = dict(plan_masks=pm, max_pages=width, sink=SINK, recent=RECENT, block_size=BS, append=True,
                  cur_k=ck.to(dev), cur_v=cv.to(dev))
        if ragged:
            a = K.decode_attention_pages_resident(q.to(dev), kh, vh, pp, pc, res, lengths=lengths, **kw)
            b = K.decode_attention_pages_ragged(q.to(dev), kh2, vh2, pp, pc, lengths, **kw)
        else:
            L = lengths0[0] + step
            a = K.decode_attention_pages_resident(q.to(dev), kh, vh, pp, pc, res, length=L, **kw)
            b = K.decode_attention_pages(q.to(dev), kh2, vh2, pp, pc, plan_masks=pm, max_pages=width, sink=SINK,
                                         recent=RECENT, block_size=BS, length=L, append_position=L,
                                         cur_k=ck.to(dev), cur_v=cv.to(dev))
        torch.cuda.synchronize()
        assert same_bits(a, b), step
        # this step's buffer == the slab's union pages at their union indices
        Ls = [L0 + step for L0 in lengths0]
        for gi in range(G):
            n = int(pc[gi])
            pages = pp[gi, :n].long().cpu()
            rows = (SINK + pages[:, None] * BS + torch.arange(BS)).reshape(-1)
            par = Ls[gi] & 1
            assert same_bits(res.k[gi, par, :n].reshape(-1, D), kh[gi][rows]), (step, gi)
            assert same_bits(res.v[gi, par, :n].reshape(-1, D), vh[gi][rows]), (step, gi)
        lengths += 1
    assert same_bits(kh, kh2) and same_bits(vh, vh2)   # the appends landed alike
    hits, union = res.stats.sum(dim=0).tolist()
    assert union > 0 and 0 < hits < union, (hits, union)


@pytest.mark.parametrize("ragged,recent", [(True, RECENT), (False, RECENT), (True, 100)])
def test_resident_windows_serve_sink_and_recent(K, dev, ragged, recent):
    """Resident sink/recent windows: after each step the host slab's copies of
    the next step's sink and recent rows are overwritten with noise, and the
    next step still equals the plain launch over the intact slab bit for bit
    (the windows come from HBM); the window buffers hold the slab's rows at
    their slots and the state names the next length.  At step 4 the window
    buffers are overwritten with noise and the state cleared instead: that
    launch reads the slab and stores the windows again.  One ragged group
    starts below the sink size and crosses it; a recent window of 100 rows
    takes a ring of 128."""
    _say(f"[resident windows] ragged={ragged} recent={recent}")
    dtype, R, k, steps = "bf16", 4, 16, 7
    lengths0 = [3000, 3000, 3000] if not ragged else [60, 2500, 3100, 4000]
    G = len(lengths0)
    Lmax = max(lengths0) + steps + 16
    keys = randn((G, Lmax, D), dtype, seed=121)
    vals = randn((G, Lmax, D), dtype, seed=122)
    kh, vh = keys.clone().pin_memory(), vals.clone().pin_memory()      # resident run, noise planted
    kh2, vh2 = keys.clone().pin_memory(), vals.clone().pin_memory()    # plain run, intact
    pmin, pmax = _metadata(keys, lengths0, dtype, dev)
    P = pmin.shape[1]
    width = min(P, R * k)
    res = K.ResidentPages(G, width, P, D, keys.dtype, dev, sink=SINK, recent=recent)
    ring = res.ring
    assert ring == (256 if recent == 256 else 128) and tuple(res.win_k.shape) == (G, SINK + ring, D)
    lengths = torch.tensor(lengths0, dtype=torch.int32, device=dev)
    g = torch.Generator().manual_seed(123)
    noise = torch.Generator().manual_seed(124)
    base = torch.randn((G, R, D), generator=g)
    for step in range(steps):
        Ls = [L0 + step for L0 in lengths0]
        kh.copy_(kh2)   # only this step's own window rows stay overwritten below
        vh.copy_(vh2)
        if step == 4:
            res.win_k.copy_(torch.randn(res.win_k.shape, generator=noise).to(res.win_k.dtype))
            res.win_v.copy_(torch.randn(res.win_v.shape, generator=noise).to(res.win_v.dtype))
            res.win_state.zero_()
        elif step > 0:
            for gi, L in enumerate(Ls):
                if L - 1 >= SINK:   # the previous launch stored the whole sink
                    kh[gi, :SINK] = torch.randn((SINK, D), generator=noise).to(kh.dtype)
                    vh[gi, :SINK] = torch.randn((SINK, D), generator=noise).to(vh.dtype)
                r0 = oracle.selection_window(L, SINK, recent)[1]   # recent - 1 history rows
                if r0 < L:
                    kh[gi, r0:L] = torch.randn((L - r0, D), generator=noise).to(kh.dtype)
                    vh[gi, r0:L] = torch.randn((L - r0, D), generator=noise).to(vh.dtype)
        q = (base + 0.15 * torch.randn((G, R, D), generator=g)).to(torch.bfloat16)
        ck, cv = randn((G, D), dtype, seed=600 + step), randn((G, D), dtype, seed=700 + step)
        pp = torch.zeros((G, width), dtype=torch.int32, device=dev)
        pm = torch.zeros((G, width), dtype=torch.uint8, device=dev)
        pc = torch.zeros((G,), dtype=torch.int32, device=dev)
        K.quest_select_ragged(q.float().to(dev), pmin, pmax, lengths, k, sink=SINK, recent=recent, block_size=BS,
                              plan_pages=pp, plan_masks=pm, plan_counts=pc)
        kw = dict(plan_masks=pm, max_pages=width, sink=SINK, recent=recent, block_size=BS, append=True,
                  cur_k=ck.to(dev), cur_v=cv.to(dev))
        if ragged:
            a = K.decode_attention_pages_resident(q.to(dev), kh, vh, pp, pc, res, lengths=lengths, **kw)
            b = K.decode_attention_pages_ragged(q.to(dev), kh2, vh2, pp, pc, lengths, **kw)
        else:
            L = Ls[0]
            a = K.decode_attention_pages_resident(q.to(dev), kh, vh, pp, pc, res, length=L, **kw)
            b = K.decode_attention_pages(q.to(dev), kh2, vh2, pp, pc, plan_masks=pm, max_pages=width, sink=SINK,
                                         recent=recent, block_size=BS, length=L, append_position=L,
                                         cur_k=ck.to(dev), cur_v=cv.to(dev))
        torch.cuda.synchronize()
        assert same_bits(a, b), step
        state = res.win_state.cpu()
        for gi, L in enumerate(Ls):
            assert same_bits(kh[gi, L], kh2[gi, L]) and same_bits(vh[gi, L], vh2[gi, L]), (step, gi)  # the append
            se = min(SINK, L)
            assert state[gi].tolist() == [L + 1, int(se == SINK)], (step, gi, state[gi].tolist())
            if se == SINK:
                assert same_bits(res.win_k[gi, :SINK], kh2[gi, :SINK]), (step, gi)
                assert same_bits(res.win_v[gi, :SINK], vh2[gi, :SINK]), (step, gi)
            rows = torch.arange(oracle.selection_window(L, SINK, recent)[1], L + 1)
            slots = SINK + (rows & (ring - 1))
            assert same_bits(res.win_k[gi, slots.to(dev)], kh2[gi, rows]), (step, gi)
            assert same_bits(res.win_v[gi, slots.to(dev)], vh2[gi, rows]), (step, gi)
        lengths += 1
    with pytest.raises(ValueError):
        K.decode_attention_pages_resident(q.to(dev), kh, vh, pp, pc, res, lengths=lengths,
                                          **dict(kw, recent=ring + 1))


@pytest.mark.parametrize("resident", [False, True])
def test_attention_fused_page_metadata(K, dev, resident):
    """The ragged page-tile attention with the page-metadata update fused in:
    40 decode steps from lengths of different page phases (one appended row
    holds a NaN) leave page_min/page_max equal to a rebuild over the final
    rows, and every step's output equals the launch without the update."""
    _say(f"[fused page metadata] resident={resident}")
    dtype, R, k, steps = "bf16", 4, 16, 40
    lengths0 = [100, 143, 200, 300]
    G = len(lengths0)
    Lmax = max(lengths0) + steps + 16
    keys = randn((G, Lmax, D), dtype, seed=131)
    vals = randn((G, Lmax, D), dtype, seed=132)
    kd, vd = keys.to(dev), vals.to(dev)
    kd2, vd2 = keys.to(dev), vals.to(dev)
    pmin, pmax = _metadata(keys, lengths0, dtype, dev)
    P = pmin.shape[1]
    width = min(P, R * k)
    res = K.ResidentPages(G, width, P, D, keys.dtype, dev) if resident else None
    lengths = torch.tensor(lengths0, dtype=torch.int32, device=dev)
    g = torch.Generator().manual_seed(133)
    for step in range(steps):
        q = torch.randn((G, R, D), generator=g).to(torch.bfloat16)
        ck, cv = randn((G, D), dtype, seed=400 + step), randn((G, D), dtype, seed=500 + step)
        if step == 11:
            ck[0, 5] = float("nan")
        pp = torch.zeros((G, width), dtype=torch.int32, device=dev)
        pm = torch.zeros((G, width), dtype=torch.uint8, device=dev)
        pc = torch.zeros((G,), dtype=torch.int32, device=dev)
        K.quest_select_ragged(q.float().to(dev), pmin, pmax, lengths, k, sink=SINK, recent=RECENT, block_size=BS,
                              plan_pages=pp, plan_masks=pm, plan_counts=pc)
        kw = dict(plan_masks=pm, max_pages=width, sink=SINK, recent=RECENT, block_size=BS, append=True,
                  cur_k=ck.to(dev), cur_v=cv.to(dev))
        if resident:
            a = K.decode_attention_pages_resident(q.to(dev), kd, vd, pp, pc, res, lengths=lengths, page_min=pmin,
                                                  page_max=pmax, **kw)
        else:
            a = K.decode_attention_pages_ragged(q.to(dev), kd, vd, pp, pc, lengths, page_min=pmin, page_max=pmax,
                                                **kw)
        b = K.decode_attention_pages_ragged(q.to(dev), kd2, vd2, pp, pc, lengths, **kw)
        torch.cuda.synchronize()
        assert same_bits(a, b), step
        lengths += 1
    assert same_bits(kd, kd2) and same_bits(vd, vd2)
    for gi, L0 in enumerate(lengths0):
        n = L0 + steps
        omin, omax, _, _, _ = oracle.build_page_metadata(to_bits(kd[gi, :n].cpu()), dtype, SINK, BS, quant=False)
        p = omin.shape[0]
        assert same_bits(pmin[gi, :p], from_bits(omin, dtype)) and same_bits(pmax[gi, :p], from_bits(omax, dtype)), gi
    with pytest.raises(ValueError):
        K.decode_attention_pages_ragged(q.to(dev), kd, vd, pp, pc, lengths, page_min=pmin, page_max=pmax,
                                        **dict(kw, append=False))


def test_twilight_select_ragged_matches_oracle(K, dev):
    """Ragged Twilight stage 2 (INT4 QK over the ragged stage-1 plan, then
    top-p and the GQA union with per-group lengths) == oracle.twilight_layer
    at each group's own length, bit for bit: B0 pages, logits, desired counts,
    each head's kept candidates and the union rows.  One group has no
    candidate page, one fewer candidate pages than B0."""
    _say("[ragged twilight select]")
    dtype, R, b0, top_p = "bf16", 4, 64, 0.9
    lengths0 = [200, 1000, 1500, 5000, 9000]
    G = len(lengths0)
    Lmax = max(lengths0) + 16
    kd = randn((G, Lmax, D), dtype, seed=141).to(dev)
    q = randn((G, R, D), "f32", seed=142).to(dev)
    P_cap = (Lmax - SINK) // BS
    pmin = torch.zeros((G, P_cap, D), dtype=kd.dtype, device=dev)
    pmax = torch.zeros_like(pmin)
    packed = torch.zeros((G, Lmax, D // 2), dtype=torch.uint8, device=dev)
    scale = torch.zeros((G, Lmax), dtype=kd.dtype, device=dev)
    minimum = torch.zeros_like(scale)
    for g, L in enumerate(lengths0):
        K.build_page_metadata(kd[g, :L], sink=SINK, block_size=BS, page_min=pmin[g], page_max=pmax[g],
                              packed=packed[g], scale=scale[g], minimum=minimum[g])
    lengths = torch.tensor(lengths0, dtype=torch.int32, device=dev)
    width = min(P_cap, R * b0)
    sel = torch.empty((G, R, b0), dtype=torch.int32, device=dev)
    pp = torch.empty((G, width), dtype=torch.int32, device=dev)
    pm = torch.empty((G, width), dtype=torch.uint8, device=dev)
    pc = torch.empty((G,), dtype=torch.int32, device=dev)
    K.quest_select_ragged(q, pmin, pmax, lengths, b0, sink=SINK, recent=RECENT, block_size=BS, sel_pages=sel,
                          plan_pages=pp, plan_masks=pm, plan_counts=pc)
    logits = K.twilight_qk(q, packed, scale, minimum, pp, pm, pc, b0, sink=SINK, block_size=BS)
    N = b0 * BS
    rows = torch.full((G, Lmax + 1), -7, dtype=torch.int32, device=dev)
    counts = torch.empty((G,), dtype=torch.int32, device=dev)
    desired = torch.empty((G, R), dtype=torch.int32, device=dev)
    hb = torch.empty((G, R, (N + 31) // 32), dtype=torch.int32, device=dev)
    K.twilight_select_ragged(logits, sel, lengths, top_p=top_p, rows=rows, row_counts=counts,
                             max_length=max(lengths0), page_capacity=P_cap, sink=SINK, recent=RECENT,
                             block_size=BS, desired=desired, head_bits=hb)
    torch.cuda.synchronize()
    keys_h = kd.cpu()
    for g, L in enumerate(lengths0):
        P = min(_cand(L), P_cap)
        kg = min(b0, P)
        n = int(counts[g])
        if kg == 0:
            sink_end, recent_start, _ = oracle.selection_window(L, SINK, RECENT)
            want = torch.cat([torch.arange(sink_end), torch.arange(recent_start, L)]).to(torch.int32)
            assert n == want.numel() and torch.equal(rows[g, :n].cpu(), want), g
            assert bool((desired[g] == 0).all()) and bool((hb[g] == 0).all()), g
            continue
        omin, omax, opk, osc, omn = oracle.build_page_metadata(to_bits(keys_h[g, :L]), dtype, SINK, BS)
        ref = oracle.twilight_layer(q[g].cpu().numpy(), omin[:P], omax[:P], opk, osc, omn, dtype, length=L, sink=SINK,
                                    recent=RECENT, block_size=BS, b0_pages=kg, top_p=top_p)
        nk = kg * BS
        assert np.array_equal(sel[g, :, :kg].cpu().numpy(), ref["pages"]), g
        assert np.array_equal(logits[g, :, :nk].cpu().numpy().view(np.uint32),
                              ref["logits"].astype(np.float32).view(np.uint32)), g
        assert np.array_equal(desired[g].cpu().numpy(), ref["desired"]), g
        bits = ((hb[g].cpu().numpy().astype(np.int64) & 0xFFFFFFFF)[:, :, None] >> np.arange(32)) & 1
        keep = bits.reshape(R, -1)[:, :nk].astype(bool)
        for r in range(R):
            assert np.array_equal(np.sort(ref["candidates"][r][keep[r]]), ref["selected"][r]), (g, r)
        assert bool((hb[g, :, (nk + 31) // 32:] == 0).all()), g
        assert n == len(ref["union"]) and np.array_equal(rows[g, :n].cpu().numpy(), ref["union"]), g


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_rows_append_fused_metadata(K, dev, dtype):
    """The rows-mode attention with the append and the INT4 + page metadata
    update fused: 40 steps from lengths of different page phases (one
    appended row holds a NaN) leave the metadata equal to a rebuild, and the
    outputs equal the launch without the update."""
    _say(f"[rows append metadata] {dtype}")
    R, steps = 4, 40
    lengths0 = [100, 143, 200, 300]
    G = len(lengths0)
    Lmax = max(lengths0) + steps + 16
    keys = randn((G, Lmax, D), dtype, seed=151)
    kd, vd = keys.to(dev), randn((G, Lmax, D), dtype, seed=152).to(dev)
    kd2, vd2 = kd.clone(), vd.clone()
    P = (Lmax - SINK) // BS
    pmin = torch.zeros((G, P, D), dtype=keys.dtype, device=dev)
    pmax = torch.zeros_like(pmin)
    packed = torch.zeros((G, Lmax, D // 2), dtype=torch.uint8, device=dev)
    scale = torch.zeros((G, Lmax), dtype=keys.dtype, device=dev)
    minimum = torch.zeros_like(scale)
    for g, L in enumerate(lengths0):
        K.build_page_metadata(kd[g, :L], sink=SINK, block_size=BS, page_min=pmin[g], page_max=pmax[g],
                              packed=packed[g], scale=scale[g], minimum=minimum[g])
    lengths = torch.tensor(lengths0, dtype=torch.int32, device=dev)
    meta = dict(sink=SINK, page_min=pmin, page_max=pmax, packed=packed, scale=scale, minimum=minimum)
    gen = torch.Generator().manual_seed(153)
    for step in range(steps):
        q = randn((G, R, D), dtype, seed=600 + step).to(dev)
        ck, cv = randn((G, D), dtype, seed=700 + step), randn((G, D), dtype, seed=800 + step)
        if step == 9:
            ck[1, 17] = float("nan")
        ck, cv = ck.to(dev), cv.to(dev)
        n = 50
        rows = torch.stack([torch.randperm(min(lengths0) + step, generator=gen)[:n].sort().values
                            for _ in range(G)]).to(torch.int32).to(dev)
        counts = torch.full((G,), n, dtype=torch.int32, device=dev)
        a = K.decode_attention_rows(q, kd, vd, rows, counts, n, cur_k=ck, cur_v=cv, append_position=lengths,
                                    metadata=meta)
        b = K.decode_attention_rows(q, kd2, vd2, rows, counts, n, cur_k=ck, cur_v=cv, append_position=lengths)
        torch.cuda.synchronize()
        assert same_bits(a, b), step
        lengths += 1
    assert same_bits(kd, kd2) and same_bits(vd, vd2)
    for g, L0 in enumerate(lengths0):
        n = L0 + steps
        omin, omax, opk, osc, omn = oracle.build_page_metadata(to_bits(kd[g, :n].cpu()), dtype, SINK, BS)
        p = omin.shape[0]
        assert same_bits(pmin[g, :p], from_bits(omin, dtype)) and same_bits(pmax[g, :p], from_bits(omax, dtype)), g
        assert np.array_equal(packed[g, :n].cpu().numpy(), opk), g
        assert same_bits(scale[g, :n], from_bits(osc, dtype)) and same_bits(minimum[g, :n], from_bits(omn, dtype)), g

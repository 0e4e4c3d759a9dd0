"""GPU parity of the bitmap form of the Quest selection and of the page-tile
attention that ranks its union from those bitmaps.

quest_select_bits must set exactly the pages of the oracle's Quest score +
top-k (bit-exact, ties to the lowest page) for every head, at one length and
at each ragged group's own length; decode_attention_pages_bits must give the
same output bits, and the same appended rows and page metadata, as the
union-plan attention over the plan of the same selection, and match float64
attention over the union rows.
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
    return oracle.selection_window(L, SINK, RECENT)[2] // BS


def _bit_rows(bits: torch.Tensor, P: int) -> np.ndarray:
    """[G, R, words] int32 -> [G, R, P] bool."""
    w = bits.cpu().numpy().view(np.uint32)
    p = np.arange(P)
    return ((w[..., p >> 5] >> (p & 31).astype(np.uint32)) & 1).astype(bool)


def _bits_tensor(K, G, R, P, dev, pad=0):
    """Selection bitmaps with a few spare words per row, prefilled with a
    pattern the kernel must overwrite."""
    words = K.sel_bits_words(P) + pad
    return torch.full((G, R, words), -1, dtype=torch.int32, device=dev)


CASES = [
    # (label, dtype, R, lengths): one length for every group, or ragged
    ("32k", "f16", 4, [32768] * 8),
    ("ragged", "bf16", 7, [40, 400, 1000, 5000, 20000, 33000]),
    ("ragged-r8", "f16", 8, [300, 4096, 17000, 33000]),
    ("96k", "bf16", 4, [96000, 95000]),  # > 4096 pages: two words per lane
]


@pytest.mark.parametrize("label,dtype,R,lengths", CASES, ids=[c[0] for c in CASES])
def test_quest_select_bits_matches_oracle(K, dev, label, dtype, R, lengths):
    """Bit p of head r's row is set exactly when the oracle's top-k of that
    head (at the group's own length) holds page p; sel_pages, when asked for
    too, equals the oracle's ascending page ids."""
    _say(f"[select bits] {label} {dtype} R={R}")
    G, k = len(lengths), 128
    Lmax = max(lengths) + 16
    keys = randn((G, Lmax, D), dtype, seed=201)
    q = randn((G, R, D), "f32", seed=202)
    one_length = len(set(lengths)) == 1
    pmin, pmax = _metadata(keys, lengths, dtype, dev)
    P = _cand(lengths[0]) if one_length else pmin.shape[1]
    pmin, pmax = pmin[:, :P], pmax[:, :P]
    bits = _bits_tensor(K, G, R, P, dev, pad=2)
    sel = torch.empty((G, R, k), dtype=torch.int32, device=dev)
    lt = None if one_length else torch.tensor(lengths, dtype=torch.int32, device=dev)
    K.quest_select_bits(q.to(dev), pmin, pmax, k, bits, lengths=lt, sel_pages=sel, sink=SINK, recent=RECENT,
                        block_size=BS)
    torch.cuda.synchronize()
    rows = _bit_rows(bits, P)
    assert bool((bits[:, :, K.sel_bits_words(P):] == -1).all()), "words past the row were written"
    pmin_h, pmax_h = to_bits(pmin), to_bits(pmax)
    for g, L in enumerate(lengths):
        Pg = min(_cand(L), P)
        kg = min(k, Pg)
        if Pg == 0:
            assert not rows[g].any(), g
            continue
        sc = oracle.quest_score(q[g:g + 1].numpy(), pmin_h[g:g + 1, :Pg], pmax_h[g:g + 1, :Pg], dtype)[0]
        want = oracle.topk_sorted(sc, kg)
        for r in range(R):
            expect = np.zeros(P, bool)
            expect[want[r]] = True
            assert np.array_equal(rows[g, r], expect), (g, r)
        assert np.array_equal(sel[g, :, :kg].cpu().numpy(), want), g
        assert bool((sel[g, :, kg:] == -1).all()), g


ATT_CASES = [
    ("32k-cur", "f16", 4, [32768] * 8, "cur_append"),
    ("32k-none", "bf16", 4, [32768] * 8, "none"),
    ("ragged-cur", "bf16", 7, [40, 400, 1000, 5000, 20000, 33000], "cur_append"),
    ("ragged-row", "f16", 4, [300, 4096, 17000, 33000], "cache_row"),
    ("96k-cur", "f16", 4, [96000, 95000], "cur_append"),
]


@pytest.mark.parametrize("label,dtype,R,lengths,decode", ATT_CASES, ids=[c[0] for c in ATT_CASES])
def test_decode_attention_pages_bits_equals_plan(K, dev, label, dtype, R, lengths, decode):
    """The bitmap-ranked attention == the union-plan attention bit for bit
    (output, appended rows, fused page metadata), and within 2e-3 abs +
    1e-2 rel of float64 attention over sink ++ union pages ++ recent ++ the
    decode token."""
    _say(f"[attention bits] {label} {dtype} R={R} decode={decode}")
    G, k = len(lengths), 128
    Lmax = max(lengths) + 16
    keys = randn((G, Lmax, D), dtype, seed=211)
    vals = randn((G, Lmax, D), dtype, seed=212)
    q = randn((G, R, D), dtype, seed=213)
    ck, cv = randn((G, D), dtype, seed=214), randn((G, D), dtype, seed=215)
    one_length = len(set(lengths)) == 1
    pmin, pmax = _metadata(keys, lengths, dtype, dev)
    P = _cand(lengths[0]) if one_length else pmin.shape[1]
    smin, smax = pmin[:, :P], pmax[:, :P]
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    width = min(P, R * k)
    pp = torch.empty((G, width), dtype=torch.int32, device=dev)
    pm = torch.empty((G, width), dtype=torch.uint8, device=dev)
    pc = torch.empty((G,), dtype=torch.int32, device=dev)
    bits = _bits_tensor(K, G, R, P, dev)
    qf = q.float().to(dev)
    if one_length:
        K.quest_select(qf, smin, smax, k, plan_pages=pp, plan_masks=pm, plan_counts=pc)
        K.quest_select_bits(qf, smin, smax, k, bits)
    else:
        K.quest_select_ragged(qf, smin, smax, lt, k, sink=SINK, recent=RECENT, block_size=BS, plan_pages=pp,
                              plan_masks=pm, plan_counts=pc)
        K.quest_select_bits(qf, smin, smax, k, bits, lengths=lt, sink=SINK, recent=RECENT, block_size=BS)
    kw = dict(max_pages=width, sink=SINK, recent=RECENT, block_size=BS)
    if decode == "cur_append":
        kw.update(append=True, cur_k=ck.to(dev), cur_v=cv.to(dev))
    else:
        kw.update(append=decode == "cache_row")
    if one_length:
        kw_bits = dict(kw, length=lengths[0])
    else:
        kw_bits = dict(kw, lengths=lt)
    outs, slabs, metas = [], [], []
    for use_bits in (False, True):
        kd, vd = keys.to(dev), vals.to(dev)
        mmin, mmax = pmin.clone(), pmax.clone()
        meta = {} if decode == "none" or one_length else dict(page_min=mmin, page_max=mmax)
        if use_bits:
            out = K.decode_attention_pages_bits(q.to(dev), kd, vd, bits, P, **kw_bits, **meta)
        elif one_length:
            pos = lengths[0] if decode != "none" else -1
            extra = {} if decode != "cur_append" else dict(cur_k=kw["cur_k"], cur_v=kw["cur_v"])
            out = K.decode_attention_pages(q.to(dev), kd, vd, pp, pc, plan_masks=pm, max_pages=width, sink=SINK,
                                           recent=RECENT, block_size=BS, length=lengths[0], append_position=pos,
                                           **extra)
        else:
            out = K.decode_attention_pages_ragged(q.to(dev), kd, vd, pp, pc, lt, plan_masks=pm, **kw, **meta)
        torch.cuda.synchronize()
        outs.append(out.cpu())
        slabs.append((kd.cpu(), vd.cpu()))
        metas.append((mmin.cpu(), mmax.cpu()))
    assert same_bits(outs[0], outs[1]), label
    assert same_bits(slabs[0][0], slabs[1][0]) and same_bits(slabs[0][1], slabs[1][1]), label
    assert same_bits(metas[0][0], metas[1][0]) and same_bits(metas[0][1], metas[1][1]), label
    # float64 over the oracle's rows (the bitmap union of each group)
    rows_b = _bit_rows(bits, P)
    ref = np.zeros((G, R, D))
    all_heads = (1 << R) - 1
    for g, L in enumerate(lengths):
        sink_end, recent_start, _ = oracle.selection_window(L, SINK, RECENT)
        union = np.flatnonzero(rows_b[g].any(axis=0))
        hm = np.zeros(union.shape[0], np.int64)
        for r in range(R):
            hm |= rows_b[g, r, union].astype(np.int64) << r
        pos = np.concatenate([np.arange(sink_end), (SINK + union[:, None] * BS + np.arange(BS)).reshape(-1),
                              np.arange(recent_start, L)]).astype(np.int64)
        m = np.concatenate([np.full(sink_end, all_heads), np.repeat(hm, BS), np.full(L - recent_start, all_heads)])
        kk, vv = keys[g, pos], vals[g, pos]
        if decode == "cur_append":
            kk, vv = torch.cat([kk, ck[g:g + 1]]), torch.cat([vv, cv[g:g + 1]])
        elif decode == "cache_row":
            kk, vv = torch.cat([kk, keys[g, L:L + 1]]), torch.cat([vv, vals[g, L:L + 1]])
        if decode != "none":
            m = np.concatenate([m, [all_heads]])
        ref[g] = oracle.decode_attention(q[g].float().numpy(), kk.float().numpy(), vv.float().numpy(),
                                         1.0 / math.sqrt(D), m.astype(np.uint8))
    got = outs[1].float().numpy().astype(np.float64)
    err = np.abs(got - ref)
    assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), f"max abs err {err.max():.3e}"


def _crafted_metadata(kind: str, G: int, P: int, dtype: str):
    """Page min/max whose scores defeat the top-k's one-pass fast path:
    hundreds of tied top scores, a NaN score, one flat row, or a few
    distinct values (boundary bins far fuller than 64 keys)."""
    lo = randn((G, P, D), dtype, seed=231)
    hi = randn((G, P, D), dtype, seed=232)
    pmin, pmax = torch.minimum(lo, hi), torch.maximum(lo, hi)
    if kind == "ties":
        # 300 copies of one strong page: the 128 best scores are all equal
        pmin[:, 5:305] = pmin[:, 4:5] * 4
        pmax[:, 5:305] = pmax[:, 4:5] * 4
    elif kind == "nan":
        pmax[:, 17, 3] = float("nan")
    elif kind == "flat":
        pmin[:] = pmin[:, :1]
        pmax[:] = pmax[:, :1]
    elif kind == "few":
        pmin[:, :] = pmin[:, torch.arange(P) % 5]
        pmax[:, :] = pmax[:, torch.arange(P) % 5]
    return pmin.contiguous(), pmax.contiguous()


@pytest.mark.parametrize("kind", ["ties", "nan", "flat", "few"])
def test_quest_select_fast_path_fallbacks(K, dev, kind):
    """Rows whose first histogram pass cannot finish the selection still
    select the oracle's pages (ties to the lowest page, NaN highest), through
    quest_select_bits and through quest_select's plan path."""
    _say(f"[select fallbacks] {kind}")
    G, R, P, k, dtype = 2, 4, 2028, 128, "f16"
    pmin, pmax = _crafted_metadata(kind, G, P, dtype)
    q = randn((G, R, D), "f32", seed=233)
    bits = _bits_tensor(K, G, R, P, dev)
    sel_b = torch.empty((G, R, k), dtype=torch.int32, device=dev)
    sel_p = torch.empty_like(sel_b)
    pp = torch.empty((G, min(P, R * k)), dtype=torch.int32, device=dev)
    pc = torch.empty((G,), dtype=torch.int32, device=dev)
    qd, dmin, dmax = q.to(dev), pmin.to(dev), pmax.to(dev)
    K.quest_select_bits(qd, dmin, dmax, k, bits, sel_pages=sel_b)
    K.quest_select(qd, dmin, dmax, k, sel_pages=sel_p, plan_pages=pp, plan_counts=pc)
    torch.cuda.synchronize()
    rows = _bit_rows(bits, P)
    sc = oracle.quest_score(q.numpy(), to_bits(pmin), to_bits(pmax), dtype)
    for g in range(G):
        want = oracle.topk_sorted(sc[g], k)
        assert np.array_equal(sel_b[g].cpu().numpy(), want), g
        assert np.array_equal(sel_p[g].cpu().numpy(), want), g
        for r in range(R):
            expect = np.zeros(P, bool)
            expect[want[r]] = True
            assert np.array_equal(rows[g, r], expect), (g, r)
        union = np.unique(want)
        assert int(pc[g]) == union.shape[0] and np.array_equal(pp[g, :union.shape[0]].cpu().numpy(), union), g

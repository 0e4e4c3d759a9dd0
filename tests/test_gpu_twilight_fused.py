"""The fused Twilight selection (twilight_select_fused) and the union-record
attention (decode_attention_union) against the oracle.

Per group, oracle.twilight_layer at the group's own length gives the B0 pages,
the INT4 QK logits, the top-p counts and each head's kept positions.  The
fused selection must reproduce the first three bit for bit, and its union
record must hold exactly the union of the heads' kept rows: one bitmap bit
per page that has a kept row, that page's rows in its 16-bit mask, nothing
else.  The attention over the record is held to 2e-3 abs + 1e-2 rel of
float64 over the oracle's rows plus the decode token, and the appended row
with its INT4 code and page metadata must equal the page-row path's bit for
bit.  Every case runs twice with new queries on a record that starts as
garbage, so a bit the score launch failed to clear would show."""

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


@pytest.fixture(scope="module")
def K():
    from headinfer import kernels

    return kernels


def _close(got, ref, what):
    got = np.asarray(got, dtype=np.float64)
    err = np.abs(got - ref)
    assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), f"{what}: max abs err {err.max():.3e}"


def _record_of(kept_pos, P, sink, bs):
    """The union record's bitmap words and per-page masks the kept token
    positions (between the sink and the recent window) give."""
    masks = np.zeros(P, np.int64)
    for p in kept_pos:
        page, i = divmod(int(p) - sink, bs)
        assert 0 <= page < P
        masks[page] |= 1 << i
    return masks


def _decode_record(rec, P):
    """(bitmap as a bool array over P pages + the bits past P, masks [P])."""
    rec = rec.astype(np.int64) & 0xFFFFFFFF
    nb = 2 * ((P + 63) // 64)
    off = (nb + 3) & ~3
    bits = np.array([(rec[p >> 5] >> (p & 31)) & 1 for p in range(32 * nb)], bool)
    masks = np.array([(rec[off + (p >> 1)] >> (16 * (p & 1))) & 0xFFFF for p in range(P)], np.int64)
    return bits, masks


class _Setup:
    def __init__(self, K, dev, G, R, Lmax, lengths, dtype=torch.bfloat16, seed=0, sink=64, recent=256, bs=16):
        self.G, self.R, self.D, self.bs, self.sink, self.recent = G, R, 128, bs, sink, recent
        D = self.D
        g = torch.Generator(device=dev).manual_seed(seed)
        self.k = (torch.randn((G, Lmax, D), generator=g, device=dev) * 1.5).to(dtype)
        self.v = torch.randn((G, Lmax, D), generator=g, device=dev).to(dtype)
        self.P = (Lmax - sink) // bs
        self.pmin = torch.zeros((G, self.P, D), dtype=dtype, device=dev)
        self.pmax = torch.zeros_like(self.pmin)
        self.packed = torch.zeros((G, Lmax, D // 2), dtype=torch.uint8, device=dev)
        self.qscale = torch.zeros((G, Lmax), dtype=dtype, device=dev)
        self.qmin = torch.zeros_like(self.qscale)
        for gi, L in enumerate(lengths):
            p = max(0, (L - sink) // bs)
            K.build_page_metadata(self.k[gi:gi + 1, :L], sink=sink, block_size=bs,
                                  page_min=self.pmin[gi:gi + 1, :p], page_max=self.pmax[gi:gi + 1, :p],
                                  packed=self.packed[gi:gi + 1, :L], scale=self.qscale[gi:gi + 1, :L],
                                  minimum=self.qmin[gi:gi + 1, :L])


def _run_case(K, dev, G, R, lengths, b0, top_p, ragged, seed):
    st = _Setup(K, dev, G, R, max(lengths) + 8, lengths, seed=seed)
    D, bs, sink, recent = st.D, st.bs, st.sink, st.recent
    L = lengths[0]
    # one length: the launch scores the pages wholly between its sink and recent windows
    P = st.P if ragged else oracle.selection_window(L, sink, recent)[2] // bs
    lens = torch.tensor(lengths, dtype=torch.int32, device=dev)
    words = K.union_record_words(P)
    rec = torch.full((G, (words + 3) & ~3), -1, dtype=torch.int32, device=dev)   # garbage: the score launch clears it
    sel = torch.zeros((G, R, b0), dtype=torch.int32, device=dev)
    logits = torch.zeros((G, R, b0 * bs), dtype=torch.float32, device=dev)
    desired = torch.zeros((G, R), dtype=torch.int32, device=dev)
    # the page-row path on a second slab copy, for the appended row and its metadata
    width = min(P, R * b0)
    ppB = torch.zeros((G, width), dtype=torch.int32, device=dev)
    pmB = torch.zeros((G, width), dtype=torch.uint8, device=dev)
    pcB = torch.zeros((G,), dtype=torch.int32, device=dev)
    selB = torch.zeros((G, R, b0), dtype=torch.int32, device=dev)
    logB = torch.zeros((G, R, b0 * bs), dtype=torch.float32, device=dev)
    slot_u = torch.zeros((G, R, b0), dtype=torch.int32, device=dev)
    prB = torch.zeros((G, width), dtype=torch.int32, device=dev)
    dB = torch.zeros((G, R), dtype=torch.int32, device=dev)
    kA, vA, kB, vB = st.k.clone(), st.v.clone(), st.k.clone(), st.v.clone()
    metaA = [t.clone() for t in (st.pmin, st.pmax, st.packed, st.qscale, st.qmin)]
    metaB = [t.clone() for t in (st.pmin, st.pmax, st.packed, st.qscale, st.qmin)]
    gen = torch.Generator(device=dev).manual_seed(seed + 1)
    for rep in range(2):
        q = (torch.randn((G, R, D), generator=gen, device=dev) * 2).to(torch.bfloat16)
        cur_k = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
        cur_v = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
        qf = q.float()
        _say(f"[fused] G={G} R={R} lengths={lengths[:3]}.. b0={b0} ragged={ragged} rep {rep}: select")
        K.twilight_select_fused(qf, metaA[0][:, :P], metaA[1][:, :P], metaA[2], metaA[3], metaA[4], b0, rec,
                                top_p=top_p, sink=sink, recent=recent, block_size=bs,
                                length=max(lengths) if ragged else L, lengths=lens if ragged else None,
                                desired=desired, sel_pages=sel, logits=logits)
        torch.cuda.synchronize()
        rec_h = rec.cpu().numpy()
        sel_h, log_h, des_h = sel.cpu().numpy(), logits.cpu().numpy(), desired.cpu().numpy()
        kept_all = []
        for gi in range(G):
            Lg = lengths[gi] if ragged else L
            sink_end, recent_start, span = oracle.selection_window(Lg, sink, recent)
            Pg = min(span // bs, P)
            bits, masks = _decode_record(rec_h[gi], P)
            b0g = min(b0, Pg)
            if b0g == 0:
                assert np.all(des_h[gi] == 0) and np.all(sel_h[gi] == -1), gi
                assert not bits.any() and not masks.any(), gi
                kept_all.append(np.concatenate([np.arange(sink_end), np.arange(recent_start, Lg)]).astype(np.int64))
                continue
            ref = oracle.twilight_layer(qf[gi].cpu().numpy(), to_bits(st.pmin[gi, :Pg]), to_bits(st.pmax[gi, :Pg]),
                                        st.packed[gi].cpu().numpy(), to_bits(st.qscale[gi]), to_bits(st.qmin[gi]),
                                        "bf16", length=Lg, sink=sink, recent=recent, block_size=bs, b0_pages=b0g,
                                        top_p=top_p)
            assert np.array_equal(sel_h[gi, :, :b0g], ref["pages"]), (rep, gi)
            assert np.all(sel_h[gi, :, b0g:] == -1), (rep, gi)
            Ng = b0g * bs
            assert np.array_equal(log_h[gi, :, :Ng].view(np.uint32), ref["logits"].astype(np.float32).view(np.uint32)), \
                (rep, gi)
            assert np.array_equal(des_h[gi], ref["desired"]), (rep, gi, des_h[gi], ref["desired"])
            sel_pos = np.unique(np.concatenate(ref["selected"]))
            want = _record_of(sel_pos, P, sink, bs)
            assert np.array_equal(masks, want), (rep, gi)
            assert np.array_equal(bits[:P], want != 0) and not bits[P:].any(), (rep, gi)
            kept_all.append(ref["union"].astype(np.int64))
        # ---- attention over the record (A) and over page rows (B) ----
        max_pages = min(P, R * b0)
        outA = K.decode_attention_union(q, kA, vA, rec, P, max_pages=max_pages, sink=sink, recent=recent,
                                        block_size=bs, lengths=lens if ragged else None, length=L, append=True,
                                        cur_k=cur_k, cur_v=cur_v, page_min=metaA[0], page_max=metaA[1],
                                        packed=metaA[2], scale=metaA[3], minimum=metaA[4])
        if ragged:
            K.quest_select_ragged(qf, metaB[0][:, :P], metaB[1][:, :P], lens, b0, sink=sink, recent=recent,
                                  block_size=bs, sel_pages=selB, plan_pages=ppB, plan_masks=pmB, plan_counts=pcB)
        else:
            K.quest_select(qf, metaB[0][:, :P], metaB[1][:, :P], b0, sel_pages=selB, plan_pages=ppB,
                           plan_masks=pmB, plan_counts=pcB)
        K.twilight_qk(qf, metaB[2], metaB[3], metaB[4], ppB, pmB, pcB, b0, sink=sink, block_size=bs, out=logB,
                      slot_u=slot_u, page_rows=prB)
        K.twilight_select_pages(logB, selB, slot_u, prB, top_p=top_p, sink=sink, recent=recent, block_size=bs,
                                length=max(lengths) if ragged else L, lengths=lens if ragged else None,
                                page_capacity=P, desired=dB)
        outB = K.decode_attention_page_rows(q, kB, vB, ppB, pcB, prB, max_pages=width, sink=sink, recent=recent,
                                            block_size=bs, lengths=lens if ragged else None, length=L, append=True,
                                            cur_k=cur_k, cur_v=cur_v, page_min=metaB[0], page_max=metaB[1],
                                            packed=metaB[2], scale=metaB[3], minimum=metaB[4])
        torch.cuda.synchronize()
        assert torch.equal(desired, dB), rep
        ref_o = np.zeros((G, R, D))
        for gi in range(G):
            kept = kept_all[gi]
            keys = torch.cat([st.k[gi, kept].float(), cur_k[gi:gi + 1].float()]).cpu().numpy()
            vals = torch.cat([st.v[gi, kept].float(), cur_v[gi:gi + 1].float()]).cpu().numpy()
            ref_o[gi] = oracle.decode_attention(qf[gi].cpu().numpy(), keys, vals, 1.0 / math.sqrt(D))
        _close(outA.float().cpu().numpy(), ref_o, f"union-record attention rep {rep}")
        _close(outB.float().cpu().numpy(), ref_o, f"page-row attention rep {rep}")
        assert torch.equal(kA.view(torch.int16), kB.view(torch.int16)) and torch.equal(vA.view(torch.int16),
                                                                                         vB.view(torch.int16))
        for a, b in zip(metaA, metaB):
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), rep
        # the next repetition reads the slab with this step's row (the oracle too)
        st.k.copy_(kA)
        st.v.copy_(vA)
        for t, a in zip((st.pmin, st.pmax, st.packed, st.qscale, st.qmin), metaA):
            t.copy_(a)
        _say(f"[fused] rep {rep} ok, desired {des_h[0].tolist()}, union pages "
             f"{[int(_decode_record(rec_h[gi], P)[0].sum()) for gi in range(G)]}")


@pytest.mark.parametrize("G,R,L,b0,top_p", [
    (4, 4, 4096, 64, 0.95),
    (2, 8, 3000, 40, 0.8),
    (3, 2, 8192, 256, 0.99),
    (2, 4, 20000, 512, 0.95),     # 8192 candidates: 16 a thread
    (2, 4, 40000, 256, 0.95),     # 2480 scored pages: 8 keys a thread in the B0 top-k
    (8, 4, 32768, 256, 0.95),     # the 32K Twilight layer's shape
])
def test_fused_selection_matches_oracle(K, dev, G, R, L, b0, top_p):
    _run_case(K, dev, G, R, [L] * G, b0, top_p, ragged=False, seed=L + G)


def test_fused_selection_matches_oracle_ragged(K, dev):
    # a group with no whole page between its windows, one with fewer pages
    # than b0, longer ones, and one past 4096 pages (16 keys a thread)
    lengths = [300, 1000, 4000, 4097, 7000, 70000]
    _run_case(K, dev, len(lengths), 4, lengths, 64, 0.95, ragged=True, seed=11)


@pytest.mark.parametrize("G,R,L,b0,top_p,fixed", [
    (4, 4, 4096, 64, 0.95, 12),
    (2, 8, 3000, 40, 0.8, 40),       # fixed == b0: every head allocated all of its candidates
    (3, 7, 9000, 100, 1.0, 30),      # seven heads, top-p 1
    (2, 4, 20000, 512, 0.95, 62),    # 8192 candidates: 16 a thread
    (8, 4, 32768, 256, 0.95, 102),   # the 32K Twilight layer, matched_budget_fraction 0.05
])
def test_fused_matched_selection_matches_oracle(K, dev, G, R, L, b0, top_p, fixed):
    """Matched budgets through the fused selection: B0 pages, logits and top-p
    counts bit for bit, the allocation (largest remainder towards fixed * 16 *
    R) equal to the oracle's, the record equal to the union of each head's
    top-allocated rows, and the attention over the record within 2e-3 abs +
    1e-2 rel of float64 over the oracle's union plus the decode token."""
    st = _Setup(K, dev, G, R, L + 8, [L] * G, seed=L + R)
    D, bs, sink, recent = st.D, st.bs, st.sink, st.recent
    P = oracle.selection_window(L, sink, recent)[2] // bs
    words = K.union_record_words(P)
    rec = torch.full((G, (words + 3) & ~3), -1, dtype=torch.int32, device=dev)   # garbage: the score launch clears it
    sel = torch.zeros((G, R, b0), dtype=torch.int32, device=dev)
    logits = torch.zeros((G, R, b0 * bs), dtype=torch.float32, device=dev)
    desired = torch.zeros((G, R), dtype=torch.int32, device=dev)
    allocated = torch.zeros((G, R), dtype=torch.int32, device=dev)
    k, v = st.k.clone(), st.v.clone()
    gen = torch.Generator(device=dev).manual_seed(L + 7)
    for rep in range(2):
        q = (torch.randn((G, R, D), generator=gen, device=dev) * 2).to(torch.bfloat16)
        cur_k = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
        cur_v = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
        qf = q.float()
        _say(f"[fused matched] G={G} R={R} L={L} b0={b0} fixed={fixed} rep {rep}")
        K.twilight_select_fused(qf, st.pmin[:, :P], st.pmax[:, :P], st.packed, st.qscale, st.qmin, b0, rec,
                                top_p=top_p, sink=sink, recent=recent, block_size=bs, length=L, desired=desired,
                                sel_pages=sel, logits=logits, budget_mode="matched", target_total=fixed * bs * R,
                                allocated=allocated)
        out = K.decode_attention_union(q, k, v, rec, P, max_pages=min(P, R * b0), sink=sink, recent=recent,
                                       block_size=bs, length=L, append=True, cur_k=cur_k, cur_v=cur_v)
        torch.cuda.synchronize()
        rec_h, sel_h, log_h = rec.cpu().numpy(), sel.cpu().numpy(), logits.cpu().numpy()
        des_h, all_h = desired.cpu().numpy(), allocated.cpu().numpy()
        ref_o = np.zeros((G, R, D))
        for gi in range(G):
            ref = oracle.twilight_layer(qf[gi].cpu().numpy(), to_bits(st.pmin[gi, :P]), to_bits(st.pmax[gi, :P]),
                                        st.packed[gi].cpu().numpy(), to_bits(st.qscale[gi]), to_bits(st.qmin[gi]),
                                        "bf16", length=L, sink=sink, recent=recent, block_size=bs, b0_pages=b0,
                                        top_p=top_p, budget_mode="matched", fixed_pages=fixed)
            assert np.array_equal(sel_h[gi], ref["pages"]), (rep, gi)
            assert np.array_equal(log_h[gi].view(np.uint32), ref["logits"].astype(np.float32).view(np.uint32)), \
                (rep, gi)
            assert np.array_equal(des_h[gi], ref["desired"]), (rep, gi, des_h[gi], ref["desired"])
            assert np.array_equal(all_h[gi], ref["allocated"]), (rep, gi, all_h[gi], ref["allocated"])
            assert all_h[gi].sum() == fixed * bs * R, (rep, gi)
            bits, masks = _decode_record(rec_h[gi], P)
            want = _record_of(np.unique(np.concatenate(ref["selected"])), P, sink, bs)
            assert np.array_equal(masks, want), (rep, gi)
            assert np.array_equal(bits[:P], want != 0) and not bits[P:].any(), (rep, gi)
            kept = ref["union"].astype(np.int64)
            keys = torch.cat([st.k[gi, kept].float(), cur_k[gi:gi + 1].float()]).cpu().numpy()
            vals = torch.cat([st.v[gi, kept].float(), cur_v[gi:gi + 1].float()]).cpu().numpy()
            ref_o[gi] = oracle.decode_attention(qf[gi].cpu().numpy(), keys, vals, 1.0 / math.sqrt(D))
        _close(out.float().cpu().numpy(), ref_o, f"matched union-record attention rep {rep}")
        assert torch.equal(k[:, L].view(torch.int16), cur_k.view(torch.int16))
        _say(f"[fused matched] rep {rep} ok, desired {des_h[0].tolist()} allocated {all_h[0].tolist()}")


def test_fused_matched_selection_ragged(K, dev):
    """Matched budgets with device lengths (the graph-captured decode): each
    group's candidate and B0 pages and its target (fixed = min(candidates,
    max(1, ceil(0.05 * eligible / 16))) pages x 16 x R) come from its own
    length; B0 pages, logits, counts, allocation and record against the
    oracle at that length, the attention against float64.  A group with no
    whole page between its windows keeps nothing."""
    lengths = [300, 3000, 4097, 9000, 20000]
    G, R, b0, top_p, frac = len(lengths), 4, 64, 0.9, 0.05
    st = _Setup(K, dev, G, R, max(lengths) + 8, lengths, seed=23)
    D, bs, sink, recent = st.D, st.bs, st.sink, st.recent
    P = st.P
    lens = torch.tensor(lengths, dtype=torch.int32, device=dev)
    words = K.union_record_words(P)
    rec = torch.full((G, (words + 3) & ~3), -1, dtype=torch.int32, device=dev)
    sel = torch.zeros((G, R, b0), dtype=torch.int32, device=dev)
    logits = torch.zeros((G, R, b0 * bs), dtype=torch.float32, device=dev)
    desired = torch.zeros((G, R), dtype=torch.int32, device=dev)
    allocated = torch.full((G, R), -7, dtype=torch.int32, device=dev)
    k, v = st.k.clone(), st.v.clone()
    gen = torch.Generator(device=dev).manual_seed(29)
    q = (torch.randn((G, R, D), generator=gen, device=dev) * 2).to(torch.bfloat16)
    cur_k = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
    cur_v = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
    qf = q.float()
    _say(f"[fused matched ragged] lengths={lengths}")
    K.twilight_select_fused(qf, st.pmin[:, :P], st.pmax[:, :P], st.packed, st.qscale, st.qmin, b0, rec, top_p=top_p,
                            sink=sink, recent=recent, block_size=bs, length=max(lengths), lengths=lens,
                            desired=desired, sel_pages=sel, logits=logits, budget_mode="matched",
                            matched_fraction=frac, allocated=allocated)
    out = K.decode_attention_union(q, k, v, rec, P, max_pages=min(P, R * b0), sink=sink, recent=recent,
                                   block_size=bs, lengths=lens, length=max(lengths), append=True, cur_k=cur_k,
                                   cur_v=cur_v)
    torch.cuda.synchronize()
    rec_h, sel_h, log_h = rec.cpu().numpy(), sel.cpu().numpy(), logits.cpu().numpy()
    des_h, all_h = desired.cpu().numpy(), allocated.cpu().numpy()
    ref_o = np.zeros((G, R, D))
    for gi, Lg in enumerate(lengths):
        sink_end, recent_start, eligible = oracle.selection_window(Lg, sink, recent)
        cand = min(eligible // bs, P)
        bits, masks = _decode_record(rec_h[gi], P)
        if cand == 0:
            assert np.all(des_h[gi] == 0) and not bits.any() and not masks.any(), gi
            assert np.all(all_h[gi] == 0), (gi, all_h[gi])   # allocated was -7: written, not left
            kept = np.concatenate([np.arange(sink_end), np.arange(recent_start, Lg)]).astype(np.int64)
        else:
            b0g = min(b0, cand)
            fixed = min(cand, max(1, math.ceil(frac * eligible / bs)))
            ref = oracle.twilight_layer(qf[gi].cpu().numpy(), to_bits(st.pmin[gi, :cand]),
                                        to_bits(st.pmax[gi, :cand]), st.packed[gi].cpu().numpy(),
                                        to_bits(st.qscale[gi]), to_bits(st.qmin[gi]), "bf16", length=Lg, sink=sink,
                                        recent=recent, block_size=bs, b0_pages=b0g, top_p=top_p,
                                        budget_mode="matched", fixed_pages=fixed)
            Ng = b0g * bs
            assert np.array_equal(sel_h[gi, :, :b0g], ref["pages"]) and np.all(sel_h[gi, :, b0g:] == -1), gi
            assert np.array_equal(log_h[gi, :, :Ng].view(np.uint32),
                                  ref["logits"].astype(np.float32).view(np.uint32)), gi
            assert np.array_equal(des_h[gi], ref["desired"]), (gi, des_h[gi], ref["desired"])
            assert np.array_equal(all_h[gi], ref["allocated"]), (gi, all_h[gi], ref["allocated"])
            want = _record_of(np.unique(np.concatenate(ref["selected"])), P, sink, bs)
            assert np.array_equal(masks, want) and np.array_equal(bits[:P], want != 0) and not bits[P:].any(), gi
            kept = ref["union"].astype(np.int64)
        keys = torch.cat([st.k[gi, kept].float(), cur_k[gi:gi + 1].float()]).cpu().numpy()
        vals = torch.cat([st.v[gi, kept].float(), cur_v[gi:gi + 1].float()]).cpu().numpy()
        ref_o[gi] = oracle.decode_attention(qf[gi].cpu().numpy(), keys, vals, 1.0 / math.sqrt(D))
    _close(out.float().cpu().numpy(), ref_o, "matched ragged union-record attention")
    _say(f"[fused matched ragged] ok, allocated {all_h.tolist()}")


def test_fused_selection_phase_one(K, dev):
    """phase 1 runs the score + INT4 QK launch alone (for timing it): the
    union records come back cleared and the counts untouched; the whole
    selection after it is the oracle's."""
    G, R, L, b0 = 2, 4, 5000, 48
    st = _Setup(K, dev, G, R, L + 8, [L] * G, seed=31)
    P = oracle.selection_window(L, st.sink, st.recent)[2] // st.bs
    words = K.union_record_words(P)
    rec = torch.full((G, (words + 3) & ~3), -1, dtype=torch.int32, device=dev)
    desired = torch.full((G, R), -5, dtype=torch.int32, device=dev)
    q = (torch.randn((G, R, 128), generator=torch.Generator(device=dev).manual_seed(32), device=dev) * 2).to(
        torch.bfloat16).float()
    args = (q, st.pmin[:, :P], st.pmax[:, :P], st.packed, st.qscale, st.qmin, b0, rec)
    kw = dict(top_p=0.95, sink=st.sink, recent=st.recent, block_size=st.bs, length=L, desired=desired)
    _say(f"[fused phase] G={G} R={R} L={L} b0={b0}")
    K.twilight_select_fused(*args, phase=1, **kw)
    torch.cuda.synchronize()
    for gi in range(G):   # the bitmap and the row masks (not the padding between them)
        bits, masks = _decode_record(rec[gi].cpu().numpy(), P)
        assert not bits.any() and not masks.any(), gi
    assert bool((desired == -5).all())
    K.twilight_select_fused(*args, **kw)
    torch.cuda.synchronize()
    for gi in range(G):
        ref = oracle.twilight_layer(q[gi].cpu().numpy(), to_bits(st.pmin[gi, :P]), to_bits(st.pmax[gi, :P]),
                                    st.packed[gi].cpu().numpy(), to_bits(st.qscale[gi]), to_bits(st.qmin[gi]), "bf16",
                                    length=L, sink=st.sink, recent=st.recent, block_size=st.bs, b0_pages=b0,
                                    top_p=0.95)
        assert np.array_equal(desired[gi].cpu().numpy(), ref["desired"])
        bits, masks = _decode_record(rec[gi].cpu().numpy(), P)
        assert np.array_equal(masks, _record_of(np.unique(np.concatenate(ref["selected"])), P, st.sink, st.bs))
    with pytest.raises(ValueError, match="phase"):
        K.twilight_select_fused(*args, phase=2, **kw)


@pytest.mark.parametrize("R", [12, 16])
def test_fused_selection_wide_group(K, dev, R):
    """More than 8 query heads per KV head through the fused selection and the
    union attention: sub-groups of at most 8 heads, their records ORed into
    the group's.  B0 pages, logits, top-p counts and the record against
    oracle.twilight_layer over all R heads (matched budgets:
    test_fused_matched_wide_group)."""
    G, L, b0 = 2, 6000, 64
    st = _Setup(K, dev, G, R, L + 8, [L] * G, seed=40 + R)
    D, bs, sink, recent = st.D, st.bs, st.sink, st.recent
    P = oracle.selection_window(L, sink, recent)[2] // bs
    words = K.union_record_words(P)
    rec = torch.full((G, (words + 3) & ~3), -1, dtype=torch.int32, device=dev)
    sel = torch.zeros((G, R, b0), dtype=torch.int32, device=dev)
    logits = torch.zeros((G, R, b0 * bs), dtype=torch.float32, device=dev)
    desired = torch.zeros((G, R), dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev).manual_seed(R)
    q = (torch.randn((G, R, D), generator=gen, device=dev) * 2).to(torch.bfloat16)
    cur_k = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
    cur_v = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
    qf = q.float()
    _say(f"[fused wide] G={G} R={R} L={L} b0={b0}")
    K.twilight_select_fused(qf, st.pmin[:, :P], st.pmax[:, :P], st.packed, st.qscale, st.qmin, b0, rec, top_p=0.9,
                            sink=sink, recent=recent, block_size=bs, length=L, desired=desired, sel_pages=sel,
                            logits=logits)
    k, v = st.k.clone(), st.v.clone()
    out = K.decode_attention_union(q, k, v, rec, P, max_pages=min(P, R * b0), sink=sink, recent=recent,
                                   block_size=bs, length=L, append=True, cur_k=cur_k, cur_v=cur_v)
    torch.cuda.synchronize()
    rec_h, sel_h, log_h, des_h = rec.cpu().numpy(), sel.cpu().numpy(), logits.cpu().numpy(), desired.cpu().numpy()
    ref_o = np.zeros((G, R, D))
    for gi in range(G):
        ref = oracle.twilight_layer(qf[gi].cpu().numpy(), to_bits(st.pmin[gi, :P]), to_bits(st.pmax[gi, :P]),
                                    st.packed[gi].cpu().numpy(), to_bits(st.qscale[gi]), to_bits(st.qmin[gi]), "bf16",
                                    length=L, sink=sink, recent=recent, block_size=bs, b0_pages=b0, top_p=0.9)
        assert np.array_equal(sel_h[gi], ref["pages"]), gi
        assert np.array_equal(log_h[gi].view(np.uint32), ref["logits"].astype(np.float32).view(np.uint32)), gi
        assert np.array_equal(des_h[gi], ref["desired"]), (gi, des_h[gi], ref["desired"])
        bits, masks = _decode_record(rec_h[gi], P)
        want = _record_of(np.unique(np.concatenate(ref["selected"])), P, sink, bs)
        assert np.array_equal(masks, want) and np.array_equal(bits[:P], want != 0) and not bits[P:].any(), gi
        kept = ref["union"].astype(np.int64)
        keys = torch.cat([st.k[gi, kept].float(), cur_k[gi:gi + 1].float()]).cpu().numpy()
        vals = torch.cat([st.v[gi, kept].float(), cur_v[gi:gi + 1].float()]).cpu().numpy()
        ref_o[gi] = oracle.decode_attention(qf[gi].cpu().numpy(), keys, vals, 1.0 / math.sqrt(D))
    _close(out.float().cpu().numpy(), ref_o, f"wide union-record attention R={R}")
    assert torch.equal(k[:, L].view(torch.int16), cur_k.view(torch.int16))


@pytest.mark.parametrize("R,ragged,target", [(12, False, "fixed"), (16, False, "fixed"), (40, False, "fixed"),
                                             (12, True, "fixed"), (12, False, "capacity"), (16, False, "tiny")])
def test_fused_matched_wide_group(K, dev, R, ragged, target):
    """Matched budgets over more than 8 query heads per KV head: the
    sub-groups' score + QK and head launches, then each sub-group's
    allocation + top-allocated launch over all R heads' counts.  B0 pages,
    logits, counts, the allocation (largest remainder over all R heads,
    summing to the group's target) and the ORed record against
    oracle.twilight_layer over all R heads; with device lengths each group's
    target from its own length (one group below the first whole page).  The
    targets also reach every candidate (heads filled to capacity) and R + 1
    (one head above one).  More than 64 heads are refused."""
    lengths = [300, 5000, 9000] if ragged else [6000, 6000]
    G, b0, top_p, frac = len(lengths), 64, 0.9, 0.05
    L = max(lengths)
    st = _Setup(K, dev, G, R, L + 8, lengths, seed=60 + R)
    D, bs, sink, recent = st.D, st.bs, st.sink, st.recent
    P = st.P if ragged else oracle.selection_window(L, sink, recent)[2] // bs
    words = K.union_record_words(P)
    rec = torch.full((G, (words + 3) & ~3), -1, dtype=torch.int32, device=dev)
    sel = torch.zeros((G, R, b0), dtype=torch.int32, device=dev)
    logits = torch.zeros((G, R, b0 * bs), dtype=torch.float32, device=dev)
    desired = torch.zeros((G, R), dtype=torch.int32, device=dev)
    allocated = torch.full((G, R), -7, dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev).manual_seed(R + 3)
    q = (torch.randn((G, R, D), generator=gen, device=dev) * 2).to(torch.bfloat16)
    cur_k = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
    cur_v = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
    qf = q.float()
    kw = dict(top_p=top_p, sink=sink, recent=recent, block_size=bs, desired=desired, sel_pages=sel, logits=logits,
              budget_mode="matched", allocated=allocated)
    fixed_one = 24
    if ragged:
        lens = torch.tensor(lengths, dtype=torch.int32, device=dev)
        kw.update(length=L, lengths=lens, matched_fraction=frac)
    else:
        lens = None
        total = {"fixed": fixed_one * bs * R, "capacity": b0 * bs * R, "tiny": R + 1}[target]
        kw.update(length=L, target_total=total)
    _say(f"[fused matched wide] G={G} R={R} lengths={lengths} b0={b0} target={target}")
    K.twilight_select_fused(qf, st.pmin[:, :P], st.pmax[:, :P], st.packed, st.qscale, st.qmin, b0, rec, **kw)
    k, v = st.k.clone(), st.v.clone()
    akw = dict(lengths=lens, length=L) if ragged else dict(length=L)
    out = K.decode_attention_union(q, k, v, rec, P, max_pages=min(P, R * b0), sink=sink, recent=recent,
                                   block_size=bs, append=True, cur_k=cur_k, cur_v=cur_v, **akw)
    torch.cuda.synchronize()
    rec_h, sel_h, log_h = rec.cpu().numpy(), sel.cpu().numpy(), logits.cpu().numpy()
    des_h, all_h = desired.cpu().numpy(), allocated.cpu().numpy()
    ref_o = np.zeros((G, R, D))
    for gi, Lg in enumerate(lengths):
        sink_end, recent_start, eligible = oracle.selection_window(Lg, sink, recent)
        cand = min(eligible // bs, P)
        bits, masks = _decode_record(rec_h[gi], P)
        if cand == 0:
            assert np.all(des_h[gi] == 0) and np.all(all_h[gi] == 0) and not bits.any() and not masks.any(), gi
            kept = np.concatenate([np.arange(sink_end), np.arange(recent_start, Lg)]).astype(np.int64)
        else:
            b0g = min(b0, cand)
            fixed = min(cand, max(1, math.ceil(frac * eligible / bs))) if ragged else fixed_one
            ref = oracle.twilight_layer(qf[gi].cpu().numpy(), to_bits(st.pmin[gi, :cand]),
                                        to_bits(st.pmax[gi, :cand]), st.packed[gi].cpu().numpy(),
                                        to_bits(st.qscale[gi]), to_bits(st.qmin[gi]), "bf16", length=Lg, sink=sink,
                                        recent=recent, block_size=bs, b0_pages=b0g, top_p=top_p,
                                        budget_mode="matched", fixed_pages=fixed,
                                        target_total=None if ragged else total)
            Ng = b0g * bs
            assert np.array_equal(sel_h[gi, :, :b0g], ref["pages"]), gi
            assert np.array_equal(log_h[gi, :, :Ng].view(np.uint32),
                                  ref["logits"].astype(np.float32).view(np.uint32)), gi
            assert np.array_equal(des_h[gi], ref["desired"]), (gi, des_h[gi], ref["desired"])
            assert np.array_equal(all_h[gi], ref["allocated"]), (gi, all_h[gi], ref["allocated"])
            assert all_h[gi].sum() == (fixed * bs * R if ragged else total), gi
            want = _record_of(np.unique(np.concatenate(ref["selected"])), P, sink, bs)
            assert np.array_equal(masks, want) and np.array_equal(bits[:P], want != 0) and not bits[P:].any(), gi
            kept = ref["union"].astype(np.int64)
        keys = torch.cat([st.k[gi, kept].float(), cur_k[gi:gi + 1].float()]).cpu().numpy()
        vals = torch.cat([st.v[gi, kept].float(), cur_v[gi:gi + 1].float()]).cpu().numpy()
        ref_o[gi] = oracle.decode_attention(qf[gi].cpu().numpy(), keys, vals, 1.0 / math.sqrt(D))
    _close(out.float().cpu().numpy(), ref_o, f"matched wide union-record attention R={R}")
    _say(f"[fused matched wide] ok, allocated {all_h[-1].tolist()}")
    if R == 12 and not ragged:
        q65 = torch.zeros((G, 65, D), dtype=torch.float32, device=dev)
        with pytest.raises(ValueError, match="at most 64 query heads"):
            K.twilight_select_fused(q65, st.pmin[:, :P], st.pmax[:, :P], st.packed, st.qscale, st.qmin, b0, rec,
                                    top_p=top_p, sink=sink, recent=recent, block_size=bs, length=L,
                                    budget_mode="matched", target_total=65 * bs)


@pytest.mark.parametrize("lengths0", [[5000, 5000, 5000], [3000, 5000, 9000]])
def test_union_attention_resident_cache(K, dev, lengths0):
    """The union-record attention over a host slab with the row-granular
    resident cache (and its sink/recent windows) == the same launch over an
    intact slab without it, bit for bit, over 6 decode steps with drifting
    queries (the fused selection rerun every step from device lengths),
    although before each step the resident run's slab copies of the rows the
    previous step kept are overwritten with noise: a row kept again is read
    from HBM.  At every step the buffer of the step's parity holds the slab's
    kept rows at their union slots; kept rows the previous step also kept are
    counted as hits, and some are."""
    from helpers import same_bits

    G, R, b0, steps, top_p = len(lengths0), 4, 64, 6, 0.9
    Lmax = max(lengths0) + steps + 8
    st = _Setup(K, dev, G, R, Lmax, lengths0, seed=71)
    D, bs, sink, recent, P = st.D, st.bs, st.sink, st.recent, st.P
    kh, vh = st.k.cpu().pin_memory(), st.v.cpu().pin_memory()        # resident run
    kh2, vh2 = st.k.cpu().pin_memory(), st.v.cpu().pin_memory()      # plain run
    width = min(P, R * b0)
    res = K.ResidentPages(G, width, P, D, torch.bfloat16, dev, sink=sink, recent=recent)
    lens = torch.tensor(lengths0, dtype=torch.int32, device=dev)
    words = K.union_record_words(P)
    rec = torch.zeros((G, (words + 3) & ~3), dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev).manual_seed(72)
    noise = torch.Generator().manual_seed(73)
    base = torch.randn((G, R, D), generator=gen, device=dev) * 2
    prev_kept = [None] * G
    _say(f"[union resident] lengths={lengths0}")
    for step in range(steps):
        Ls = [L0 + step for L0 in lengths0]
        # the resident run's slab copies of the rows the previous step kept
        # turn to noise: a row kept again must come from HBM
        kh.copy_(kh2)
        vh.copy_(vh2)
        for gi in range(G):
            if prev_kept[gi] is not None and len(prev_kept[gi]):
                n = len(prev_kept[gi])
                kh[gi, prev_kept[gi]] = torch.randn((n, D), generator=noise).to(kh.dtype)
                vh[gi, prev_kept[gi]] = torch.randn((n, D), generator=noise).to(vh.dtype)
        q = (base + 0.3 * torch.randn((G, R, D), generator=gen, device=dev)).to(torch.bfloat16)
        cur_k = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
        cur_v = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
        K.twilight_select_fused(q.float(), st.pmin[:, :P], st.pmax[:, :P], st.packed, st.qscale, st.qmin, b0, rec,
                                top_p=top_p, sink=sink, recent=recent, block_size=bs, length=Lmax - 8,
                                lengths=lens)
        kw = dict(max_pages=width, sink=sink, recent=recent, block_size=bs, lengths=lens, length=Lmax - 8,
                  append=True, cur_k=cur_k, cur_v=cur_v)
        a = K.decode_attention_union(q, kh, vh, rec, P, resident=res, **kw)
        b = K.decode_attention_union(q, kh2, vh2, rec, P, **kw)
        torch.cuda.synchronize()
        assert same_bits(a, b), step
        rec_h = rec.cpu().numpy()
        for gi, L in enumerate(Ls):
            assert same_bits(kh[gi, L], kh2[gi, L]) and same_bits(vh[gi, L], vh2[gi, L]), (step, gi)  # the append
            bits, masks = _decode_record(rec_h[gi], P)
            pages = np.flatnonzero(bits[:P])
            par = L & 1
            kept = []
            for u, p in enumerate(pages[:width]):
                rows = [r for r in range(bs) if (masks[p] >> r) & 1]
                pos = torch.tensor([sink + int(p) * bs + r for r in rows])
                kept.append(pos)
                assert same_bits(res.k[gi, par, u, rows], kh2[gi, pos]), (step, gi, u)
                assert same_bits(res.v[gi, par, u, rows], vh2[gi, pos]), (step, gi, u)
            prev_kept[gi] = torch.cat(kept) if kept else None
        lens += 1
    hits, union = res.stats.sum(dim=0).tolist()
    _say(f"[union resident] hit rows {hits} of {union}")
    assert union > 0 and 0 < hits < union, (hits, union)
    with pytest.raises(ValueError, match="at most 8 query heads"):
        K.decode_attention_union(torch.zeros((G, 12, D), dtype=torch.bfloat16, device=dev), kh, vh, rec, P,
                                 resident=res, **kw)

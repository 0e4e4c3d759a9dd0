"""The Twilight page-row path against the row-list path.

The row-list path (twilight_select(_ragged) + decode_attention_rows) builds the
GQA union as a list of token positions; the page-row path
(twilight_qk with slot_u / page_rows, twilight_select_pages,
decode_attention_page_rows) publishes each kept row as a bit of its B0 union
page and attends the union pages with those masks.  Both must keep the same
rows (compared as sets, exactly), give the same top-p counts, write the same
appended row and INT4 / page metadata (bit for bit), and attend within
2e-3 abs + 1e-2 rel of each other and of float64 over the oracle's rows.
Every case runs twice with new queries, so a row bit left from the first
call would show."""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

import oracle
from helpers import randn, to_bits

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


def _kept_from_page_rows(pp, pc, pr, L, sink, recent, bs):
    """Token positions the page-row plan attends (without the decode token)."""
    sink_end, recent_start, _ = oracle.selection_window(L, sink, recent)
    out = list(range(sink_end))
    for u in range(int(pc)):
        m = int(pr[u]) & 0xFFFFFFFF
        base = sink + int(pp[u]) * bs
        out += [base + i for i in range(bs) if (m >> i) & 1]
    out += list(range(recent_start, L))
    return np.array(sorted(out), np.int64)


class _Setup:
    def __init__(self, K, dev, G, R, Lmax, lengths, b0, dtype=torch.bfloat16, seed=0, sink=64, recent=256, bs=16):
        self.G, self.R, self.D, self.bs, self.sink, self.recent, self.b0 = G, R, 128, bs, sink, recent, b0
        self.lengths = lengths
        D = self.D
        g = torch.Generator(device=dev).manual_seed(seed)
        self.k = (torch.randn((G, Lmax, D), generator=g, device=dev) * 1.5).to(dtype)
        self.v = torch.randn((G, Lmax, D), generator=g, device=dev).to(dtype)
        npages = (Lmax - sink) // bs
        self.P = npages
        self.pmin = torch.empty((G, npages, D), dtype=dtype, device=dev)
        self.pmax = torch.empty_like(self.pmin)
        self.packed = torch.empty((G, Lmax, D // 2), dtype=torch.uint8, device=dev)
        self.qscale = torch.empty((G, Lmax), dtype=dtype, device=dev)
        self.qmin = torch.empty_like(self.qscale)
        L0 = min(lengths)
        K.build_page_metadata(self.k[:, :L0], sink=sink, block_size=bs, page_min=self.pmin[:, : (L0 - sink) // bs],
                              page_max=self.pmax[:, : (L0 - sink) // bs], packed=self.packed[:, :L0],
                              scale=self.qscale[:, :L0], minimum=self.qmin[:, :L0])
        # groups longer than the shortest one: metadata and INT4 rows over their own prompts
        for gi, L in enumerate(lengths):
            if L > L0:
                p = (L - sink) // bs
                K.build_page_metadata(self.k[gi:gi + 1, :L], sink=sink, block_size=bs,
                                      page_min=self.pmin[gi:gi + 1, :p], page_max=self.pmax[gi:gi + 1, :p],
                                      packed=self.packed[gi:gi + 1, :L], scale=self.qscale[gi:gi + 1, :L],
                                      minimum=self.qmin[gi:gi + 1, :L])


def _run_case(K, dev, G, R, lengths, b0, top_p, ragged, seed):
    st = _Setup(K, dev, G, R, max(lengths) + 8, lengths, b0, seed=seed)
    D, bs, sink, recent = st.D, st.bs, st.sink, st.recent
    N = b0 * bs
    L = lengths[0]
    # one length: the pages wholly between the sink and the recent window
    P_use = st.P if ragged else oracle.selection_window(L, sink, recent)[2] // bs
    width = min(P_use, R * b0)
    lens = torch.tensor(lengths, dtype=torch.int32, device=dev)
    # two slab copies: each path appends its own decode row and metadata
    kA, vA, kB, vB = st.k.clone(), st.v.clone(), st.k.clone(), st.v.clone()
    metaA = [t.clone() for t in (st.pmin, st.pmax, st.packed, st.qscale, st.qmin)]
    metaB = [t.clone() for t in (st.pmin, st.pmax, st.packed, st.qscale, st.qmin)]
    sel = torch.zeros((G, R, b0), dtype=torch.int32, device=dev)
    pp = torch.zeros((G, width), dtype=torch.int32, device=dev)
    pm = torch.zeros((G, width), dtype=torch.uint8, device=dev)
    pc = torch.zeros((G,), dtype=torch.int32, device=dev)
    logits = torch.zeros((G, R, N), dtype=torch.float32, device=dev)
    slot_u = torch.full((G, R, b0), -1, dtype=torch.int32, device=dev)
    page_rows = torch.full((G, width), -1, dtype=torch.int32, device=dev)   # garbage: QK must clear it
    rows = torch.zeros((G, max(lengths) + 2), dtype=torch.int32, device=dev)
    counts = torch.zeros((G,), dtype=torch.int32, device=dev)
    dA = torch.zeros((G, R), dtype=torch.int32, device=dev)
    dB = torch.zeros((G, R), dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev).manual_seed(seed + 1)
    for rep in range(2):
        q = (torch.randn((G, R, D), generator=gen, device=dev) * 2).to(torch.bfloat16)
        cur_k = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
        cur_v = torch.randn((G, D), generator=gen, device=dev).to(torch.bfloat16)
        qf = q.float()
        if ragged:
            K.quest_select_ragged(qf, st.pmin, st.pmax, lens, b0, sink=sink, recent=recent, block_size=bs,
                                  sel_pages=sel, plan_pages=pp, plan_masks=pm, plan_counts=pc)
        else:
            K.quest_select(qf, st.pmin[:, :P_use], st.pmax[:, :P_use], b0, sel_pages=sel, plan_pages=pp,
                           plan_masks=pm, plan_counts=pc)
        K.twilight_qk(qf, metaA[2], metaA[3], metaA[4], pp, pm, pc, b0, sink=sink, block_size=bs, out=logits,
                      slot_u=slot_u, page_rows=page_rows)
        # path A: the union row list
        if ragged:
            K.twilight_select_ragged(logits, sel, lens, top_p=top_p, rows=rows, row_counts=counts,
                                     max_length=max(lengths), page_capacity=st.P, sink=sink, recent=recent,
                                     block_size=bs, desired=dA)
            appA = lens
        else:
            K.twilight_select(logits, sel, top_p=top_p, budget_mode="dynamic", rows=rows, row_counts=counts,
                              desired=dA, sink=sink, recent=recent, block_size=bs, length=L)
            appA = L
        max_rows = min(max(lengths), sink + R * N + recent)
        outA = K.decode_attention_rows(q, kA, vA, rows, counts, max_rows, cur_k=cur_k, cur_v=cur_v,
                                       append_position=appA,
                                       metadata=dict(sink=sink, page_min=metaA[0], page_max=metaA[1],
                                                     packed=metaA[2], scale=metaA[3], minimum=metaA[4]))
        # path B: page rows
        K.twilight_select_pages(logits, sel, slot_u, page_rows, top_p=top_p, sink=sink, recent=recent, block_size=bs,
                                length=max(lengths) if ragged else L, lengths=lens if ragged else None,
                                page_capacity=st.P, desired=dB)
        outB = K.decode_attention_page_rows(q, kB, vB, pp, pc, page_rows, max_pages=width, sink=sink, recent=recent,
                                            block_size=bs, lengths=lens if ragged else None, length=L, append=True,
                                            cur_k=cur_k, cur_v=cur_v, page_min=metaB[0], page_max=metaB[1],
                                            packed=metaB[2], scale=metaB[3], minimum=metaB[4])
        torch.cuda.synchronize()
        assert torch.equal(dA, dB), rep
        rows_h, counts_h = rows.cpu().numpy(), counts.cpu().numpy()
        pp_h, pc_h, pr_h = pp.cpu().numpy(), pc.cpu().numpy(), page_rows.cpu().numpy()
        ref = np.zeros((G, R, D))
        for gi in range(G):
            Lg = lengths[gi] if ragged else L
            n = int(counts_h[gi])
            listed = np.sort(rows_h[gi, :n].astype(np.int64))
            if not ragged:
                listed = listed[listed != L]      # the row list also names the appended row
            kept = _kept_from_page_rows(pp_h[gi], pc_h[gi], pr_h[gi], Lg, sink, recent, bs)
            assert np.array_equal(listed, kept), (rep, gi)
            keys = torch.cat([st.k[gi, kept].float(), cur_k[gi:gi + 1].float()]).cpu().numpy()
            vals = torch.cat([st.v[gi, kept].float(), cur_v[gi:gi + 1].float()]).cpu().numpy()
            ref[gi] = oracle.decode_attention(q[gi].float().cpu().numpy(), keys, vals, 1.0 / math.sqrt(D))
        _close(outA.float().cpu().numpy(), ref, f"rows path rep {rep}")
        _close(outB.float().cpu().numpy(), ref, f"page-row path rep {rep}")
        # the appended row and its metadata, bit for bit
        assert torch.equal(kA.view(torch.int16), kB.view(torch.int16)) and torch.equal(vA.view(torch.int16),
                                                                                         vB.view(torch.int16))
        for a, b in zip(metaA, metaB):
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), rep
        # both caches now hold this step's row: the next repetition attends from the same slabs again
        st.k.copy_(kA)
        st.v.copy_(vA)
        kB.copy_(kA)
        vB.copy_(vA)
        _say(f"[page rows] G={G} R={R} ragged={ragged} rep {rep} ok, kept {[int(c) for c in counts_h]}")


@pytest.mark.parametrize("G,R,L,b0,top_p", [(4, 4, 4096, 64, 0.95), (2, 8, 3000, 40, 0.8), (3, 2, 8192, 256, 0.99),
                                             (2, 4, 20000, 1024, 0.95)])   # 16384 candidates: two pages per thread
def test_page_rows_match_row_list(K, dev, G, R, L, b0, top_p):
    _run_case(K, dev, G, R, [L] * G, b0, top_p, ragged=False, seed=L + G)


def test_page_rows_match_row_list_ragged(K, dev):
    # a group with no whole page between its sink and recent windows, one
    # with fewer pages than b0, and longer ones
    lengths = [300, 1000, 4000, 4097, 7000]
    _run_case(K, dev, len(lengths), 4, lengths, 64, 0.95, ragged=True, seed=11)

"""GPU parity of the first-layer kernels against the CPU oracle.

Bit-exact: page metadata, INT4 pack, Quest scores (reference order), top-k
page ids (ties -> lowest index), the fused row plan, row gather (HBM and
zero-copy pinned host) and append.  Attention: within 2e-3 abs + 1e-2 rel of
a float64 reference.  All calls go through the C ABI via headinfer.kernels.
"""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

import oracle
from helpers import TORCH_DT, from_bits, minmax_pages, randn, same_bits, to_bits

pytestmark = pytest.mark.gpu


def _say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def K():
    from headinfer import kernels

    return kernels


# ------------------------------------------------------------ metadata
META_CASES = [
    ("f16", 4103, 128, 64, 16),
    ("bf16", 4103, 128, 64, 16),
    ("f32", 1030, 128, 64, 16),
    ("bf16", 16, 4, 1, 1),
    ("f16", 63, 128, 64, 16),
    ("bf16", 200, 256, 5, 7),
    ("f16", 100, 6, 3, 4),
]


@pytest.mark.parametrize("dtype,T,D,sink,bs", META_CASES)
def test_page_metadata_bit_exact(K, dev, dtype, T, D, sink, bs):
    _say(f"[metadata] {dtype} T={T} D={D} sink={sink} bs={bs}")
    keys = randn((T, D), dtype, seed=T + D)
    keys[min(3, T - 1)] = 0.5  # constant row (scale clamps; fp16 scale underflows)
    if T > 10:
        keys[7, 1] = float("nan")
        keys[9, :] = -0.0
        keys[9, 2] = 0.0
    P = (T - sink) // bs if T > sink else 0
    kd = keys.to(dev)
    pmin = torch.empty((max(P, 1), D), dtype=keys.dtype, device=dev)
    pmax = torch.empty_like(pmin)
    packed = torch.empty((T, D // 2), dtype=torch.uint8, device=dev)
    scale = torch.empty((T,), dtype=keys.dtype, device=dev)
    minimum = torch.empty_like(scale)
    K.build_page_metadata(kd, sink=sink, block_size=bs, page_min=pmin, page_max=pmax, packed=packed, scale=scale,
                          minimum=minimum)
    torch.cuda.synchronize()
    omin, omax, opk, osc, omn = oracle.build_page_metadata(to_bits(keys), dtype, sink, bs)
    assert np.array_equal(packed.cpu().numpy(), opk)
    assert same_bits(scale, from_bits(osc, dtype))
    assert same_bits(minimum, from_bits(omn, dtype))
    if P:
        assert same_bits(pmin[:P], from_bits(omin, dtype))
        assert same_bits(pmax[:P], from_bits(omax, dtype))


@pytest.mark.parametrize(
    "dtype,D,sink,bs,host",
    [("f16", 128, 64, 16, False), ("bf16", 128, 64, 16, True), ("f32", 64, 5, 7, False), ("bf16", 6, 3, 4, True)],
)
def test_update_page_metadata_matches_rebuild(K, dev, dtype, D, sink, bs, host):
    """Prompt build, then one decode-time update per appended row (crossing
    several page boundaries) == a rebuild over all rows, bit for bit."""
    _say(f"[metadata update] {dtype} D={D} sink={sink} bs={bs} host={host}")
    E = 3
    T0 = sink + 5 * bs + 3
    Lmax = T0 + 3 * bs + 2
    keys = randn((E, Lmax, D), dtype, seed=D + bs)
    keys[1, T0 + bs, 1] = float("nan")  # a NaN in a page completed during decode
    keys[2, T0 + 2, :] = 0.25            # a constant decode row
    kd = keys.to(dev)
    slab = keys.clone().pin_memory() if host else kd
    P = (Lmax - sink) // bs
    pmin = torch.full((E, P, D), 7.0, dtype=keys.dtype, device=dev)
    pmax = torch.full_like(pmin, 7.0)
    packed = torch.zeros((E, Lmax, D // 2), dtype=torch.uint8, device=dev)
    scale = torch.zeros((E, Lmax), dtype=keys.dtype, device=dev)
    minimum = torch.zeros_like(scale)
    K.build_page_metadata(kd[:, :T0], sink=sink, block_size=bs, page_min=pmin, page_max=pmax, packed=packed,
                          scale=scale, minimum=minimum)
    for pos in range(T0, Lmax):
        for e0, n in ((0, 1), (1, E - 1)):
            K.update_page_metadata(slab, first_entry=e0, n_entries=n, position=pos, sink=sink, block_size=bs,
                                   page_min=pmin, page_max=pmax, packed=packed, scale=scale, minimum=minimum)
    torch.cuda.synchronize()
    for e in range(E):
        omin, omax, opk, osc, omn = oracle.build_page_metadata(to_bits(keys[e]), dtype, sink, bs)
        assert omin.shape[0] == P
        assert same_bits(pmin[e], from_bits(omin, dtype)) and same_bits(pmax[e], from_bits(omax, dtype)), e
        assert np.array_equal(packed[e].cpu().numpy(), opk), e
        assert same_bits(scale[e], from_bits(osc, dtype)) and same_bits(minimum[e], from_bits(omn, dtype)), e


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
def test_int4_round_trip_bound(K, dev, dtype):
    """scripts/test_twilight_offload_cache_v1.py:82-89 on the GPU path."""
    keys = randn((17, 128), dtype, seed=7)
    packed, scale, minimum = K.affine_int4_pack(keys.to(dev))
    restored = K.affine_int4_dequantize(packed, scale, minimum)
    assert packed.shape == (17, 64) and restored.shape == (17, 128)
    err = (restored.cpu() - keys.float()).abs().amax(dim=-1)
    assert torch.isfinite(restored).all()
    assert torch.all(err <= scale.cpu().float() / 2 + 1e-6)
    odq = oracle.int4_dequantize(packed.cpu().numpy(), to_bits(scale), to_bits(minimum), dtype)
    assert np.array_equal(restored.cpu().numpy().view(np.uint32), odq.view(np.uint32))


# --------------------------------------------------------- Quest score
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("pages", [17, 186, 465, 1000, 2025, 2048])
def test_quest_score_and_topk_bit_exact(K, dev, dtype, pages):
    """Cases of scripts/test_twilight_fused_quest_v1.py:11-25 (seed 20260911)."""
    _say(f"[quest] {dtype} pages={pages}")
    g = torch.Generator().manual_seed(20260911 + pages)
    for kind in ("bf16", "fp32", "exponents"):
        q = torch.randn((8, 3, 128), generator=g)
        if kind == "bf16":
            q = q.bfloat16().float()
        if kind == "exponents":
            q = q * torch.exp2(torch.randint(-12, 12, q.shape, generator=g).float())
        lo, hi = minmax_pages(dtype, 8, pages, 128, seed=pages * 3 + len(kind))
        got = K.fused_quest_score(q.to(dev), lo.to(dev), hi.to(dev))
        ref = oracle.quest_score(q.numpy(), to_bits(lo), to_bits(hi), dtype)
        assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32)), kind
        k = min(pages, 512)
        idx = K.topk_sorted(got, k)
        assert np.array_equal(idx.cpu().numpy(), oracle.topk_sorted(ref, k)), kind


@pytest.mark.parametrize("value", [0.0, 1.0, -1.0])
def test_quest_score_tie_cases(K, dev, value):
    """scripts/test_twilight_fused_quest_v1.py:26-34: constant q, lo=-2, hi=1."""
    q = torch.full((8, 3, 128), value)
    lo = torch.full((8, 513, 128), -2.0, dtype=torch.bfloat16)
    hi = torch.ones_like(lo)
    got = K.fused_quest_score(q.to(dev), lo.to(dev), hi.to(dev))
    ref = oracle.quest_score(q.numpy(), to_bits(lo), to_bits(hi), "bf16")
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    idx = K.topk_sorted(got, 512)
    assert np.array_equal(idx.cpu().numpy(), np.broadcast_to(np.arange(512), (8, 3, 512)))


def test_topk_ties_nan_negzero(K, dev):
    g = torch.Generator().manual_seed(5)
    s = torch.randint(-3, 4, (16, 1000), generator=g).float()
    s[0, 10] = float("nan")
    s[1, :] = 0.0
    s[1, ::3] = -0.0
    s[2, :] = float("-inf")
    s[3, 500:] = float("inf")
    for k in (1, 7, 64, 999, 1000):
        got = K.topk_sorted(s.to(dev), k)
        assert np.array_equal(got.cpu().numpy(), oracle.topk_sorted(s.numpy(), k)), k


@pytest.mark.parametrize("P", [5, 1000, 2028, 2048, 4076, 8169, 8192])
def test_topk_distributions(K, dev, P):
    """Score shapes that exercise every selection pass: heavy outliers that
    stretch the linear range, clusters of equal values at the boundary (more
    than a block of equal candidates), tiny ranges, and mixed signs."""
    _say(f"[topk dist] P={P}")
    g = torch.Generator().manual_seed(P)
    rows = []
    rows.append(torch.randn(P, generator=g))
    out = torch.randn(P, generator=g)
    out[torch.randperm(P, generator=g)[: max(1, P // 100)]] *= 1e4  # planted outliers
    rows.append(out)
    rows.append(torch.randint(0, 3, (P,), generator=g).float())  # large equal clusters
    rows.append(1.0 + torch.randn(P, generator=g) * 1e-6)  # range of a few ulps
    rows.append(torch.randn(P, generator=g) * torch.exp2(torch.randint(-60, 60, (P,), generator=g).float()))
    rows.append(torch.full((P,), 2.5).index_put_((torch.tensor([P // 2]),), torch.tensor(3.0)))
    s = torch.stack(rows)
    for k in sorted({1, min(P, 7), min(P, 128), max(1, P // 2), min(P, 300), P}):
        got = K.topk_sorted(s.to(dev), k)
        assert np.array_equal(got.cpu().numpy(), oracle.topk_sorted(s.numpy(), k)), k
        # the contiguous vector-load path (P % 4 == 0, aligned rows) and the scalar path both run
        wide = torch.zeros((s.shape[0], P + 3))
        wide[:, :P] = s
        got2 = K.topk_sorted(wide.to(dev)[:, :P], k)
        assert np.array_equal(got2.cpu().numpy(), oracle.topk_sorted(s.numpy(), k)), ("strided", k)


# ------------------------------------------------------ fused selection
@pytest.mark.parametrize(
    "dtype,G,R,L,sink,recent,bs,frac",
    [
        ("f16", 8, 4, 4096, 64, 256, 16, 0.0625),   # 4K-context layer, k = 16 pages
        ("f16", 8, 4, 32768, 64, 256, 16, 0.0625),  # 32K-context layer, k = 128 pages
        ("bf16", 4, 7, 20000, 64, 256, 16, 0.05),
        ("bf16", 2, 3, 16, 1, 2, 1, 0.5),
        ("f32", 3, 8, 1000, 10, 20, 8, 0.2),
    ],
)
def test_quest_select_row_plan(K, dev, dtype, G, R, L, sink, recent, bs, frac):
    _say(f"[quest_select] {dtype} G={G} R={R} L={L}")
    D = 128 if L > 16 else 4
    cand, k = oracle.quest_budget(L, sink, recent, bs, frac, (L - sink) // bs)
    P = cand
    lo, hi = minmax_pages(dtype, G, P, D, seed=L)
    q = randn((G, R, D), "f32", seed=L + 1)
    stride = L + 1
    rows = torch.full((G, stride), -7, dtype=torch.int32, device=dev)
    masks = torch.zeros((G, stride), dtype=torch.uint8, device=dev)
    counts = torch.zeros((G,), dtype=torch.int32, device=dev)
    sel = torch.empty((G, R, k), dtype=torch.int32, device=dev)
    scores = torch.empty((G, R, P), dtype=torch.float32, device=dev)
    pw = min(P, R * k)
    ppages = torch.full((G, pw), -3, dtype=torch.int32, device=dev)
    pmasks = torch.zeros((G, pw), dtype=torch.uint8, device=dev)
    pcounts = torch.zeros((G,), dtype=torch.int32, device=dev)
    for it in range(3):  # repeated: the arrival counters must be reset by the kernel
        K.quest_select(q.to(dev), lo.to(dev), hi.to(dev), k, scores=scores, sel_pages=sel, plan_pages=ppages,
                       plan_masks=pmasks, plan_counts=pcounts, rows=rows, row_masks=masks, row_counts=counts,
                       sink=sink, recent=recent, block_size=bs, length=L, append_position=L)
        torch.cuda.synchronize()
    ref_scores = oracle.quest_score(q.numpy(), to_bits(lo), to_bits(hi), dtype)
    assert np.array_equal(scores.cpu().numpy().view(np.uint32), ref_scores.view(np.uint32))
    ref_sel = oracle.topk_sorted(ref_scores, k)
    assert np.array_equal(sel.cpu().numpy(), ref_sel)
    for g in range(G):
        r_rows, r_masks = oracle.quest_row_plan(ref_sel[g], P, sink, recent, bs, L, L)
        n = int(counts[g])
        assert n == len(r_rows)
        assert np.array_equal(rows[g, :n].cpu().numpy(), r_rows)
        assert np.array_equal(masks[g, :n].cpu().numpy(), r_masks)
        # union plan: the pages any head selected, ascending, with the heads' bitmask
        union = np.unique(ref_sel[g])
        nu = int(pcounts[g])
        assert nu == len(union) and np.array_equal(ppages[g, :nu].cpu().numpy(), union)
        want = [sum(1 << r for r in range(R) if p in ref_sel[g, r]) for p in union]
        assert np.array_equal(pmasks[g, :nu].cpu().numpy(), np.array(want, np.uint8))


# ------------------------------------------------------------ attention
def _attn_ref(q, kc, vc, rows, masks, cur_k, cur_v, scale):
    out = []
    for g in range(q.shape[0]):
        keys = kc[g][rows[g]].float().numpy()
        vals = vc[g][rows[g]].float().numpy()
        m = masks[g] if masks is not None else None
        if cur_k is not None:
            keys = np.concatenate([keys, cur_k[g : g + 1].float().numpy()])
            vals = np.concatenate([vals, cur_v[g : g + 1].float().numpy()])
            if m is not None:
                m = np.concatenate([m, np.array([255], np.uint8)])
        out.append(oracle.decode_attention(q[g].float().numpy(), keys, vals, scale, m))
    return np.stack(out)


def _close(got, ref, atol=2e-3, rtol=1e-2):
    got = got.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    ok = err <= atol + rtol * np.abs(ref)
    assert ok.all(), f"max abs err {err.max():.3e}"


@pytest.mark.parametrize(
    "dtype,G,R,D,L,n_rows,masked,cur",
    [
        ("f16", 8, 4, 128, 32768, 2368, True, True),
        ("bf16", 8, 4, 128, 32768, 8512, False, True),
        ("bf16", 4, 7, 128, 5000, 700, True, True),
        ("f16", 2, 1, 64, 3000, 333, False, False),
        ("f32", 3, 8, 128, 2000, 1000, True, True),
        ("bf16", 2, 3, 4, 32, 9, True, True),
        ("f16", 2, 2, 256, 1000, 129, False, True),
        ("bf16", 8, 4, 128, 32768, 6000, "sparse", True),
    ],
)
def test_decode_attention_rows(K, dev, dtype, G, R, D, L, n_rows, masked, cur):
    _say(f"[attention rows] {dtype} G={G} R={R} D={D} rows={n_rows}")
    g0 = torch.Generator().manual_seed(L + n_rows)
    kc = randn((G, L, D), dtype, seed=1)
    vc = randn((G, L, D), dtype, seed=2)
    q = randn((G, R, D), dtype, seed=3)
    rows = torch.stack([torch.randperm(L, generator=g0)[:n_rows].sort().values for _ in range(G)]).to(torch.int32)
    counts = torch.tensor([n_rows - 5 * g if n_rows > 5 * G else n_rows for g in range(G)], dtype=torch.int32)
    masks = None
    if masked == "sparse":
        # each head sees about one row in 300: most blocks hold no visible row
        # for some head, which must contribute nothing (not NaN) to the merge
        masks = (torch.rand((G, n_rows, R), generator=g0) < 1 / 300).to(torch.uint8)
        masks = (masks << torch.arange(R, dtype=torch.uint8)).sum(-1).to(torch.uint8)
        masks[:, -1] = (1 << R) - 1
    elif masked:
        masks = torch.randint(0, 1 << R, (G, n_rows), generator=g0).to(torch.uint8)
        masks[:, -1] = (1 << R) - 1  # each head sees at least one row
    ck = randn((G, D), dtype, seed=4) if cur else None
    cv = randn((G, D), dtype, seed=5) if cur else None
    scale = 1.0 / math.sqrt(D)
    out = K.decode_attention_rows(q.to(dev), kc.to(dev), vc.to(dev), rows.to(dev), counts.to(dev), n_rows,
                                  row_masks=None if masks is None else masks.to(dev),
                                  cur_k=None if ck is None else ck.to(dev), cur_v=None if cv is None else cv.to(dev))
    torch.cuda.synchronize()
    ref_rows = [rows[g, : int(counts[g])].long().numpy() for g in range(G)]
    ref_masks = None if masks is None else [masks[g, : int(counts[g])].numpy() for g in range(G)]
    ref = _attn_ref(q, kc, vc, ref_rows, ref_masks, ck, cv, scale)
    _close(out, ref)


@pytest.mark.parametrize(
    "dtype,G,R,D,L,n_rows",
    [
        ("bf16", 8, 4, 128, 32768, 9500),   # the Twilight 32K union
        ("f16", 3, 7, 64, 3000, 400),
        ("f32", 2, 3, 128, 2000, 1000),
        ("bf16", 2, 3, 4, 32, 9),
    ],
)
def test_decode_attention_rows_append(K, dev, dtype, G, R, D, L, n_rows):
    """The fused append writes cur_k/cur_v to the row and nothing else, and the
    attention output is bit-identical to the launch without it."""
    _say(f"[attention rows append] {dtype} G={G} R={R} D={D} rows={n_rows}")
    g0 = torch.Generator().manual_seed(L + 7 * n_rows)
    Lmax = L + 3
    kc = randn((G, Lmax, D), dtype, seed=11).to(dev)
    vc = randn((G, Lmax, D), dtype, seed=12).to(dev)
    q = randn((G, R, D), dtype, seed=13).to(dev)
    rows = torch.stack([torch.randperm(L, generator=g0)[:n_rows].sort().values for _ in range(G)]).to(torch.int32)
    counts = torch.tensor([max(1, n_rows - 3 * g) for g in range(G)], dtype=torch.int32)
    ck = randn((G, D), dtype, seed=14).to(dev)
    cv = randn((G, D), dtype, seed=15).to(dev)
    rows, counts = rows.to(dev), counts.to(dev)
    plain = K.decode_attention_rows(q, kc, vc, rows, counts, n_rows, cur_k=ck, cur_v=cv)
    k0, v0 = kc.clone(), vc.clone()
    fused = K.decode_attention_rows(q, kc, vc, rows, counts, n_rows, cur_k=ck, cur_v=cv, append_position=L)
    torch.cuda.synchronize()
    assert torch.equal(fused, plain)
    k0[:, L], v0[:, L] = ck, cv
    assert torch.equal(kc, k0) and torch.equal(vc, v0)
    # per-group rows from the device (one beyond the entry: skipped)
    at = torch.tensor([L + 1 + (g % 2) for g in range(G)], dtype=torch.int32)
    at[-1] = Lmax + 5
    ragged = K.decode_attention_rows(q, kc, vc, rows, counts, n_rows, cur_k=ck, cur_v=cv,
                                     append_position=at.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(ragged, plain)
    for g in range(G):
        if int(at[g]) < Lmax:
            k0[g, int(at[g])], v0[g, int(at[g])] = ck[g], cv[g]
    assert torch.equal(kc, k0) and torch.equal(vc, v0)
    with pytest.raises(ValueError):
        K.decode_attention_rows(q, kc, vc, rows, counts, n_rows, append_position=L)
    with pytest.raises(ValueError):
        K.decode_attention_rows(q, kc, vc, rows, counts, n_rows, cur_k=ck, cur_v=cv, append_position=Lmax)


@pytest.mark.parametrize(
    "dtype,G,R,D,L,k,sink,recent,bs,masked",
    [
        ("f16", 8, 4, 128, 32768, 128, 64, 256, 16, True),   # the 32K Quest layer
        ("bf16", 4, 7, 128, 20000, 60, 64, 256, 16, True),
        ("bf16", 3, 2, 64, 3000, 20, 10, 30, 12, False),     # page size not a power of two
        ("f32", 2, 3, 128, 1500, 8, 1, 2, 8, True),
        ("f16", 2, 2, 6, 400, 5, 4, 9, 4, True),             # generic head dim
    ],
)
def test_decode_attention_pages(K, dev, dtype, G, R, D, L, k, sink, recent, bs, masked):
    """Attention over a union page plan == attention over its expanded rows."""
    _say(f"[attention pages] {dtype} G={G} R={R} D={D} L={L} k={k}")
    g0 = torch.Generator().manual_seed(L + k)
    sink_end, recent_start, eligible = oracle.selection_window(L, sink, recent)
    P = eligible // bs
    Lmax = L + 1
    kc = randn((G, Lmax, D), dtype, seed=41)
    vc = randn((G, Lmax, D), dtype, seed=42)
    q = randn((G, R, D), dtype, seed=43)
    max_pages = min(P, R * k)
    pages = torch.zeros((G, max_pages), dtype=torch.int32)
    pm = torch.zeros((G, max_pages), dtype=torch.uint8)
    counts = torch.zeros((G,), dtype=torch.int32)
    for g in range(G):
        n = int(torch.randint(1, max_pages + 1, (1,), generator=g0))
        pages[g, :n] = torch.randperm(P, generator=g0)[:n].sort().values.to(torch.int32)
        pm[g, :n] = torch.randint(1, 1 << R, (n,), generator=g0).to(torch.uint8)
        counts[g] = n
    kd, vd = kc.to(dev), vc.to(dev)
    out = K.decode_attention_pages(q.to(dev), kd, vd, pages.to(dev), counts.to(dev),
                                   plan_masks=pm.to(dev) if masked else None, max_pages=max_pages, sink=sink,
                                   recent=recent, block_size=bs, length=L, append_position=L)
    # the fused form: the decode token from cur_k/cur_v, appended to row L in the same launch
    ck, cv = randn((G, D), dtype, seed=44), randn((G, D), dtype, seed=45)
    out2 = K.decode_attention_pages(q.to(dev), kd, vd, pages.to(dev), counts.to(dev),
                                    plan_masks=pm.to(dev) if masked else None, max_pages=max_pages, sink=sink,
                                    recent=recent, block_size=bs, length=L, append_position=L,
                                    cur_k=ck.to(dev), cur_v=cv.to(dev))
    torch.cuda.synchronize()
    assert same_bits(kd[:, L], ck) and same_bits(vd[:, L], cv)
    assert same_bits(kd[:, :L], kc[:, :L]) and same_bits(vd[:, :L], vc[:, :L])
    ref = np.zeros((G, R, D))
    ref2 = np.zeros((G, R, D))
    all_heads = (1 << R) - 1
    for g in range(G):
        n = int(counts[g])
        pg = pages[g, :n].long()
        rows = torch.cat([torch.arange(sink_end), (sink + pg[:, None] * bs + torch.arange(bs)).reshape(-1),
                          torch.arange(recent_start, L), torch.tensor([L])])
        m = None
        if masked:
            m = torch.cat([torch.full((sink_end,), all_heads), pm[g, :n].long().repeat_interleave(bs),
                           torch.full((L - recent_start + 1,), all_heads)]).to(torch.uint8).numpy()
        ref[g] = oracle.decode_attention(q[g].float().numpy(), kc[g, rows].float().numpy(),
                                         vc[g, rows].float().numpy(), 1.0 / math.sqrt(D), m)
        kc[g, L], vc[g, L] = ck[g], cv[g]
        ref2[g] = oracle.decode_attention(q[g].float().numpy(), kc[g, rows].float().numpy(),
                                          vc[g, rows].float().numpy(), 1.0 / math.sqrt(D), m)
    _close(out, ref)
    _close(out2, ref2)


@pytest.mark.parametrize(
    "dtype,G,R,L,n_pages,decode,masked",
    [
        ("bf16", 2, 8, 700, 12, "cur_append", False),  # 8 heads, unmasked
        ("f16", 3, 1, 500, 11, "cur_append", True),    # one head
        ("f16", 2, 2, 900, 30, "cache_row", True),     # decode token read from cache row L
        ("bf16", 2, 3, 1200, 40, "none", True),        # no decode token
        ("f16", 2, 5, 1000, 25, "cur_only", True),     # decode token attended, not appended
        ("bf16", 2, 4, 40, 0, "cur_append", False),    # context inside the sink window
        ("f16", 2, 4, 300, 0, "cur_append", True),     # sink + recent only
        ("f16", 3, 4, 70000, 1100, "cur_append", True),  # two batches per wavefront
    ],
)
def test_decode_attention_page_tiles(K, dev, dtype, G, R, L, n_pages, decode, masked):
    """16-row pages at D = 128 (the page-tile kernel): partial sink and recent
    tiles, every decode-token form, R from 1 to 8, plan counts above the plan
    width (clamped), against float64 over the expanded rows."""
    _say(f"[attention page tiles] {dtype} G={G} R={R} L={L} pages={n_pages} decode={decode}")
    D, sink, recent, bs = 128, 64, 256, 16
    g0 = torch.Generator().manual_seed(L + R)
    sink_end, recent_start, eligible = oracle.selection_window(L, sink, recent)
    P = eligible // bs
    width = max(1, n_pages)
    Lmax = L + 2
    kc = randn((G, Lmax, D), dtype, seed=61)
    vc = randn((G, Lmax, D), dtype, seed=62)
    q = randn((G, R, D), dtype, seed=63)
    pages = torch.zeros((G, width), dtype=torch.int32)
    pm = torch.zeros((G, width), dtype=torch.uint8)
    counts = torch.zeros((G,), dtype=torch.int32)
    for g in range(G):
        n = min(n_pages, P) if g == 0 else int(torch.randint(0, min(n_pages, P) + 1, (1,), generator=g0))
        if n:
            pages[g, :n] = torch.randperm(P, generator=g0)[:n].sort().values.to(torch.int32)
            pm[g, :n] = torch.randint(1, 1 << R, (n,), generator=g0).to(torch.uint8)
        counts[g] = n
    counts_dev = counts.clone()
    if n_pages:
        counts_dev[0] = width + 5  # beyond the plan width: the launch covers `width` pages
    ck, cv = randn((G, D), dtype, seed=64), randn((G, D), dtype, seed=65)
    kd, vd = kc.to(dev), vc.to(dev)
    kw = dict(plan_masks=pm.to(dev) if masked else None, max_pages=width if n_pages else 0, sink=sink,
              recent=recent, block_size=bs, length=L)
    if decode == "cur_append":
        kw.update(append_position=L, cur_k=ck.to(dev), cur_v=cv.to(dev))
    elif decode == "cur_only":
        kw.update(append_position=-1, cur_k=ck.to(dev), cur_v=cv.to(dev))
    elif decode == "cache_row":
        kw.update(append_position=L)
    else:
        kw.update(append_position=-1)
    out = K.decode_attention_pages(q.to(dev), kd, vd, pages.to(dev), counts_dev.to(dev), **kw)
    torch.cuda.synchronize()
    if decode == "cur_append":
        assert same_bits(kd[:, L], ck) and same_bits(vd[:, L], cv)
    else:
        assert same_bits(kd[:, L], kc[:, L]) and same_bits(vd[:, L], vc[:, L])
    all_heads = (1 << R) - 1
    ref = np.zeros((G, R, D))
    for g in range(G):
        n = int(counts[g])
        pg = pages[g, :n].long()
        keys = [kc[g, :sink_end], kc[g, (sink + pg[:, None] * bs + torch.arange(bs)).reshape(-1)],
                kc[g, recent_start:L]]
        vals = [vc[g, :sink_end], vc[g, (sink + pg[:, None] * bs + torch.arange(bs)).reshape(-1)],
                vc[g, recent_start:L]]
        m = [np.full(sink_end, all_heads), pm[g, :n].long().repeat_interleave(bs).numpy() if masked
             else np.full(n * bs, all_heads), np.full(L - recent_start, all_heads)]
        if decode.startswith("cur"):
            keys.append(ck[g:g + 1])
            vals.append(cv[g:g + 1])
        elif decode == "cache_row":
            keys.append(kc[g, L:L + 1])
            vals.append(vc[g, L:L + 1])
        if decode != "none":
            m.append(np.array([all_heads]))
        ref[g] = oracle.decode_attention(q[g].float().numpy(), torch.cat(keys).float().numpy(),
                                         torch.cat(vals).float().numpy(), 1.0 / math.sqrt(D),
                                         np.concatenate(m).astype(np.uint8))
    _close(out, ref)


@pytest.mark.parametrize("dtype,B,Hk,R,D", [("bf16", 8, 1, 4, 128), ("f16", 3, 2, 3, 128), ("bf16", 5, 1, 1, 4)])
def test_decode_attention_varlen(K, dev, dtype, B, Hk, R, D):
    _say(f"[attention varlen] {dtype} B={B} Hk={Hk} R={R} D={D}")
    g0 = torch.Generator().manual_seed(B * 100 + D)
    lens = torch.randint(1, 3000 if D > 4 else 40, (B,), generator=g0)
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = lens.cumsum(0)
    total = int(cu[-1])
    k = randn((total, Hk, D), dtype, seed=11)
    v = randn((total, Hk, D), dtype, seed=12)
    q = randn((B, Hk * R, D), dtype, seed=13)
    for window in (-1, 100):
        out = K.decode_attention_varlen(q.to(dev), k.to(dev), v.to(dev), cu.to(dev), int(lens.max()),
                                        window_left=window)
        torch.cuda.synchronize()
        ref = np.zeros((B, Hk * R, D))
        for b in range(B):
            s0, s1 = int(cu[b]), int(cu[b + 1])
            if window >= 0:
                s0 = max(s0, s1 - (window + 1))
            for h in range(Hk):
                ref[b, h * R:(h + 1) * R] = oracle.decode_attention(
                    q[b, h * R:(h + 1) * R].float().numpy(), k[s0:s1, h].float().numpy(),
                    v[s0:s1, h].float().numpy(), 1.0 / math.sqrt(D))
        _close(out, ref)


# ------------------------------------------------------- rows movement
@pytest.mark.parametrize("host", [False, True])
def test_gather_rows_bit_exact(K, dev, host):
    _say(f"[gather] host={host}")
    g0 = torch.Generator().manual_seed(123)
    rows_total, D = 10000, 128
    k = randn((rows_total, D), "bf16", seed=21)
    v = randn((rows_total, D), "bf16", seed=22)
    if host:
        k, v = k.pin_memory(), v.pin_memory()
    else:
        k, v = k.to(dev), v.to(dev)
    for n in (0, 1, 8192):
        src = torch.randint(rows_total, (n,), generator=g0)
        dk = torch.empty((n, D), dtype=torch.bfloat16, device=dev)
        dv = torch.empty_like(dk)
        flag = torch.zeros((), dtype=torch.int32, device=dev)
        K.gather_rows(k, v, src.to(dev), dk, dv, error_flag=flag)
        torch.cuda.synchronize()
        assert int(flag) == 0
        assert same_bits(dk, k.cpu()[src]) and same_bits(dv, v.cpu()[src])
    # scatter into a direct layout with gaps, plus one invalid source row
    src = torch.tensor([5, 9999, 0, 10000, -1, 77])
    dst = torch.tensor([0, 1, 3, 4, 5, 6])
    dk = torch.zeros((8, D), dtype=torch.bfloat16, device=dev)
    dv = torch.zeros_like(dk)
    flag = torch.zeros((), dtype=torch.int32, device=dev)
    K.gather_rows(k, v, src.to(dev), dk, dv, dst.to(dev), error_flag=flag)
    torch.cuda.synchronize()
    assert int(flag) == 1
    kc = k.cpu()
    for s, d in ((5, 0), (9999, 1), (0, 3), (77, 6)):
        assert same_bits(dk[d], kc[s])
    assert (dk[[2, 4, 5, 7]].float() == 0).all()


@pytest.mark.parametrize("host", [False, True])
def test_append_kv(K, dev, host):
    E, Lmax, D = 6, 40, 128
    dk = torch.zeros((E, Lmax, D), dtype=torch.float16)
    dv = torch.zeros_like(dk)
    if host:
        dk, dv = dk.pin_memory(), dv.pin_memory()
    else:
        dk, dv = dk.to(dev), dv.to(dev)
    nk = randn((3, D), "f16", seed=31).to(dev)
    nv = randn((3, D), "f16", seed=32).to(dev)
    K.append_kv(nk, nv, dk, dv, first_entry=2, position=17)
    torch.cuda.synchronize()
    assert same_bits(dk[2:5, 17], nk.cpu()) and same_bits(dv[2:5, 17], nv.cpu())
    assert float(dk.cpu().float().abs().sum()) == float(nk.cpu().float().abs().sum())


@pytest.mark.parametrize("dtype,G,R,D,L,k", [("f16", 8, 4, 128, 32768, 128), ("bf16", 3, 2, 64, 3000, 20)])
def test_decode_attention_pages_phases(K, dev, dtype, G, R, D, L, k):
    """Phase 1 (split-K partials) then phase 2 (merge) == the single call, bit for bit."""
    _say(f"[attention phases] {dtype} G={G} L={L}")
    g0 = torch.Generator().manual_seed(L + 7)
    sink, recent, bs = 64, 256, 16
    sink_end, recent_start, eligible = oracle.selection_window(L, sink, recent)
    P = eligible // bs
    mp = min(P, R * k)
    pages = torch.zeros((G, mp), dtype=torch.int32)
    pm = torch.zeros((G, mp), dtype=torch.uint8)
    counts = torch.zeros((G,), dtype=torch.int32)
    for g in range(G):
        n = int(torch.randint(1, mp + 1, (1,), generator=g0))
        pages[g, :n] = torch.randperm(P, generator=g0)[:n].sort().values.to(torch.int32)
        pm[g, :n] = torch.randint(1, 1 << R, (n,), generator=g0).to(torch.uint8)
        counts[g] = n
    kc = randn((G, L + 1, D), dtype, seed=51).to(dev)
    vc = randn((G, L + 1, D), dtype, seed=52).to(dev)
    q = randn((G, R, D), dtype, seed=53).to(dev)
    args = (q, kc, vc, pages.to(dev), counts.to(dev))
    kw = dict(plan_masks=pm.to(dev), max_pages=mp, sink=sink, recent=recent, block_size=bs, length=L,
              append_position=L)
    full = K.decode_attention_pages(*args, **kw)
    split = torch.empty_like(full)
    K.decode_attention_pages(*args, **kw, out=split, phase=1)
    K.decode_attention_pages(*args, **kw, out=split, phase=2)
    torch.cuda.synchronize()
    assert same_bits(full, split)
